// pa_attn.h - kernel argument blocks and launchers of the phone-attn HIP kernels (internal to libpa_hip.so).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pa_hip {

constexpr int MAXP = 64;   // pages per attention launch (more are split over several launches into one slot array)

enum { CFG_DECODE = 0, CFG_MID = 1, CFG_VERIFY = 2, CFG_PREFILL = 3 };   // 16 / 64 / 128 / 128 rows per workgroup

struct AttnArgs {
    const uint8_t * kp[MAXP];       // page base (key 0, head 0) of K / V
    const uint8_t * vp[MAXP];
    uint32_t pstart[MAXP + 1];      // key prefix: page p holds keys [pstart[p], pstart[p+1]) of the call
    uint32_t n_pages, n_chunks, chunk, n_items;   // chunk = keys per workgroup; n_items = chunks x heads x row blocks
    uint32_t rs, hb, nkv;
    uint32_t rows;                  // real query rows per KV head
    uint32_t qr;                    // padded rows per KV head in q16 / the slots
    uint32_t nrb;                   // row blocks per KV head
    uint32_t slot0;                 // slot of chunk 0 of this launch
    float s_mul;                    // factor from the dot to base-2 logits (scale * log2 e, or log2 e)
    uint32_t hilo;                  // 1: the query's lo half is non-zero (ggml mode, quantized K)
    uint32_t q16_lo;                // offset of the lo half from q16 (elements)
    const _Float16 * q16;           // hi [nkv][qr][hd], lo at q16 + q16_lo
    float * po;                     // [slot][nkv][qr][hd]
    float2 * pml;                   // [slot][nkv][qr]: (max in base-2 units, sum)
};

struct MergeArgs {
    const float * po;
    const float2 * pml;
    float * O, * m, * l;            // [nkv][rows][hd], [nkv][rows]
    uint32_t n_slots, nkv, qr, rows;
};

struct QprepArgs {
    const float * q;                // [nkv][rows][hd] fp32
    _Float16 * q16;                 // hi [nkv][qr][hd], lo at q16 + q16_lo
    uint32_t q16_lo;
    uint32_t nkv, rows, qr, hd, qmode, fmt;
    float scale;
};

hipError_t launch_attention(int hd, int fmt, int cfg, const AttnArgs & a, uint32_t grid, hipStream_t st);
hipError_t launch_merge(int hd, const MergeArgs & a, hipStream_t st);
hipError_t launch_qprep(const QprepArgs & a, hipStream_t st);
hipError_t launch_quantize(int fmt, const float * x, void * y, int64_t n, hipStream_t st);
void cfg_geometry(int cfg, int hd, int & rows_per_wg, int & nb);

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

}  // namespace pa_hip
