// pa_decode.hip - decode partial attention for up to 8 query rows per KV head (one token x GQA 8), q8_0 / q4_0 K and V,
// ggml query rounding, head_dim 128 (gfx950).
//
// One workgroup = one pair of KV heads x one group of 32-key tiles (every G-th tile of the call), two waves (one per
// head) that share each tile. HBM traffic is coalesced: per tile wave 0 reads the pair's contiguous 16-byte aligned slice of every K
// row (2 x 136 bytes for q8_0) and wave 1 the same of V, with 16-byte loads along the rows, two tiles ahead in
// registers; both write their half raw into LDS. From there each lane takes its key's K quants as the MFMA operand and
// copies the V quants into its wave's aligned tile, both read as whole aligned 16-byte chunks and byte-aligned in
// registers (q8_0 blocks are 34 bytes, so their quants sit at 2-byte alignment; unaligned LDS reads run at a fraction
// of the aligned rate). Rows are 16-byte multiples apart, so eight consecutive keys' chunks fall in distinct LDS banks.
//
// Per 32-key tile a wave computes:
//   QK on the int8 matrix cores, exactly ggml's integer block dots. One v_mfma_i32_16x16x64_i8 per 32-dim quant block
//   covers all 32 keys: its 16 output rows are the 8 query rows twice (rows 0-7 against keys 0-15, rows 8-15 against
//   keys 16-31), with the query block placed in the first or second 32 bytes of the 64-byte reduction so the two halves
//   never mix (lane (g, n) of the K operand holds key 16*(g/2) + n, bytes 16*(g%2) .. +15 of the block). A q4_0 block is
//   used as its unsigned nibbles; the MFMA accumulator starts at -8 * (sum of the query block's quants). The block dot is
//   then scaled in fp32 by the query block scale (times softmax scale and log2 e) and the key block scale, as ggml's
//   vec_dot does per block.
//
//   Online softmax in base 2 with a reference max that moves only when a score exceeds it by more than 2^PMAX_LOG2;
//   the exact running max is tracked alongside. Lane (g, n) holds key 16*(g/2) + n for rows 4*(g%2) .. +3.
//
//   PV on the fp16 matrix cores: O^T (16 dims x rows) += V^T (16 dims x 32 keys) . P'^T (32 keys x rows), where P' = P *
//   (V block scale of that key), one P' per V block. V^T comes from the wave's aligned V tile by the transposing
//   ds_read_b64_tr_b8 (lane (g, n): dim n, keys 8g .. 8g+7), turned into fp16 as the subnormal (q + 128) * 2^-24 with one
//   xor and four byte permutes; a second MFMA with the constant -128 * 2^-24 (q4_0: -136 * 2^-24, nibbles stored
//   unsigned) removes the bias exactly, so the accumulator holds (sum P' q) * 2^-24. P' is transposed from the score
//   layout through LDS with ds_read_b64_tr_b16.
//
// Reference roles: pa_attn_big + pa_big_load (pa-metal.mm:379-487: per (row tile, KV head, key chunk), dequant a K/V
// block, S = QK^T, online softmax, O = alpha O + PV, write a split-K slot); ggml's vec_dot_q8_0_q8_0 / q4_0_q8_0 block
// arithmetic for the scores (restated in oracle/pa_oracle.c, orc_attn_ggml).
#include "pa_attn.h"
#include "pa_common.h"
#include <hip/hip_ext.h>

namespace pa_hip {

typedef int dec_v4i __attribute__((ext_vector_type(4)));
typedef int dec_v2i __attribute__((ext_vector_type(2)));
typedef __fp16 dec_h4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
#define DEC_LDS __attribute__((address_space(3)))

constexpr int DEC_HD = 128;
constexpr int DEC_NKB = DEC_HD / 32;      // quant blocks per head row
constexpr int DEC_ND = DEC_HD / 16;       // 16-dim blocks of O^T
constexpr int DEC_VST = DEC_HD + 16;      // LDS bytes per V tile row (16 bytes of padding: conflict-free tr_b8 reads)
constexpr int DEC_PBLK = 32 * 16;         // LDS bytes of one P' block: [32 keys][8 rows] fp16
constexpr int DEC_QBLK = 8 * 32 + 16;     // LDS bytes of one query block table: [8 rows][2 halves][16 bytes] + zero slot
constexpr int DEC_WLDS = 32 * DEC_VST + DEC_NKB * DEC_PBLK + DEC_NKB * DEC_QBLK + 2 * DEC_NKB * 8 * 4;
                                          // per wave: V tile, P' tiles, query tables, query scales + q4_0 sums
constexpr float PMAX_LOG2 = 6.0f;         // p <= 2^6 between rescales (P' = p * d_v stays finite for |d_v| < 1023)
constexpr int DEC_PF = 2;                 // tiles whose raw bytes are in flight in registers per wave (3: no faster)

template <int FMT> struct DecGeom {
    static constexpr int BB = FMT == 1 ? 34 : 18;          // bytes per quant block
    static constexpr int HB = BB * DEC_NKB;                // bytes per head in a key row (136 / 72, both 8 mod 16)
    static constexpr int SL = 2 * HB;                      // a head pair's slice of a key row (272 / 144, 16-aligned)
    static constexpr int NCH = SL / 16;                    // 16-byte chunks per slice (17 / 9)
};

// Cross-lane reductions on the VALU (no LDS): DPP within a 16-lane row (quad swaps, then rotations by 4 and 8), then
// v_permlane32_swap, which hands each lane the pair (value of lane l % 32, value of lane l % 32 + 32).
template <int CTRL> __device__ __forceinline__ float dec_dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float dec_rowmax32(float v) {   // max over the 32 lanes that share (g % 2): n bits and g / 2
    v = fmaxf(v, dec_dpp<0xb1>(v));                          // quad_perm [1,0,3,2]
    v = fmaxf(v, dec_dpp<0x4e>(v));                          // quad_perm [2,3,0,1]
    v = fmaxf(v, dec_dpp<0x124>(v));                         // row_ror:4
    v = fmaxf(v, dec_dpp<0x128>(v));                         // row_ror:8
    const auto t = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v), false, false);
    return fmaxf(__builtin_bit_cast(float, (unsigned) t[0]), __builtin_bit_cast(float, (unsigned) t[1]));
}
__device__ __forceinline__ float dec_rowsum32(float v) {
    v += dec_dpp<0xb1>(v);
    v += dec_dpp<0x4e>(v);
    v += dec_dpp<0x124>(v);
    v += dec_dpp<0x128>(v);
    const auto t = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v), false, false);
    return __builtin_bit_cast(float, (unsigned) t[0]) + __builtin_bit_cast(float, (unsigned) t[1]);
}

// LDS written by some lanes of a wave and read by others: DS instructions of one wave execute in order, so a
// wavefront-scope fence (no instruction, only a compiler ordering point) is enough.
__device__ __forceinline__ void dec_wave_sync() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); }

// 16 bytes at byte offset S (compile-time) inside the 32 bytes of two consecutive aligned 16-byte LDS chunks x, y:
// unaligned LDS reads run at a fraction of the aligned rate, so the rows are read as whole chunks and byte-aligned here
template <int S> __device__ __forceinline__ pa_u4 dec_align(const pa_u4 & x, const pa_u4 & y) {
    const uint32_t d[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
    constexpr int W = S / 4, B = S % 4;
    pa_u4 r;
    #pragma unroll
    for (int j = 0; j < 4; j++) r[j] = B ? __builtin_amdgcn_alignbyte(d[W + j + 1], d[W + j], B) : d[W + j];
    return r;
}
template <int S> __device__ __forceinline__ uint32_t dec_scale_bits(const pa_u4 & x) {   // the 16 bits at byte S - 2 of x
    const uint32_t d[4] = {x.x, x.y, x.z, x.w};
    constexpr int P = S - 2;
    return (d[P / 4] >> (8 * (P % 4))) & 0xffffu;
}

// One quant block of one key from the wave's raw rows (16-byte aligned, the head's bytes at OFF): the 16 bytes the
// lane needs (q8_0: half hh of the 32 quants; q4_0: all 16 nibble bytes) and the block's fp16 scale (bits), read as
// whole aligned chunks. The scale sits in the 2 bytes before the quants: inside the first chunk read by the half-0 lane
// unless the quants start a chunk (then a 16-bit read).
template <int FMT, int OFF, int B>
__device__ __forceinline__ void dec_block(const char * row, int hh, pa_u4 & q, uint32_t & sc) {
    using G = DecGeom<FMT>;
    constexpr int o = OFF + G::BB * B + 2, S = o & 15, C0 = o >> 4;
    const char * c = row + 16 * C0 + (FMT == 1 ? 16 * hh : 0);
    const pa_u4 x = *(const pa_u4 *) c;
    if constexpr (S == 0) {
        q = x;
        sc = *(const uint16_t *) (row + o - 2);
    } else {
        const pa_u4 y = *(const pa_u4 *) (c + 16);
        q = dec_align<S>(x, y);
        sc = S >= 2 ? dec_scale_bits<(S >= 2 ? S : 2)>(x) : 0u;
        if constexpr (FMT == 1) {                                    // the half-1 lane takes the half-0 lane's scale
            const auto t = __builtin_amdgcn_permlane16_swap(sc, sc, false, false);
            sc = t[0];
        }
    }
}

// the wave's tile from its raw rows: this lane's K operands and scales, V scales, and the V quants into the aligned tile
// [key][32 * block] (q4_0: nibbles unpacked to bytes, element order)
template <int FMT, int OFF>
__device__ __forceinline__ void dec_unpack(const char * krow, const char * vrow, uint8_t * vdst, int hh, dec_v4i (&kq)[DEC_NKB],
                                           float (&dkf)[DEC_NKB], pa_h2 (&dvh)[DEC_NKB]) {
    #pragma unroll
    for (int b = 0; b < DEC_NKB; b++) {
        pa_u4 qk, qv;
        uint32_t sk, sv;
        switch (b) {
            case 0: dec_block<FMT, OFF, 0>(krow, hh, qk, sk); dec_block<FMT, OFF, 0>(vrow, hh, qv, sv); break;
            case 1: dec_block<FMT, OFF, 1>(krow, hh, qk, sk); dec_block<FMT, OFF, 1>(vrow, hh, qv, sv); break;
            case 2: dec_block<FMT, OFF, 2>(krow, hh, qk, sk); dec_block<FMT, OFF, 2>(vrow, hh, qv, sv); break;
            default: dec_block<FMT, OFF, 3>(krow, hh, qk, sk); dec_block<FMT, OFF, 3>(vrow, hh, qv, sv); break;
        }
        kq[b] = __builtin_bit_cast(dec_v4i, qk);
        dkf[b] = pa_f16_bits_to_f32((uint16_t) sk);
        const _Float16 dv = __builtin_bit_cast(_Float16, (uint16_t) sv);
        dvh[b] = (pa_h2){dv, dv};
        if constexpr (FMT == 2) {
            const int sh = 4 * hh;
            qv = (pa_u4){(qv.x >> sh) & 0x0f0f0f0fu, (qv.y >> sh) & 0x0f0f0f0fu, (qv.z >> sh) & 0x0f0f0f0fu, (qv.w >> sh) & 0x0f0f0f0fu};
        }
        *(pa_u4 *) (vdst + 32 * b + 16 * hh) = qv;
    }
}

// LDS-only workgroup barrier: the vector-memory loads in flight (the next tiles) are not waited for
__device__ __forceinline__ void dec_lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int FMT>
__global__ __launch_bounds__(128, 2) void dec_kernel(const AttnArgs a) {
    using G = DecGeom<FMT>;
    constexpr int TCH = 32 * G::NCH;                                 // 16-byte chunks of one tensor's tile (544 / 288)
    constexpr int CPL = (TCH + 63) / 64;                             // per lane of the wave that loads it (9 / 5)
    constexpr int RAW = 2 * TCH * 16;                                // the tile's raw pair slices: K rows, then V rows
    constexpr int LDS = RAW + 2 * DEC_WLDS;
    __shared__ __attribute__((aligned(16))) char smem[LDS];

    // ---- which (group, head pair): the call's 32-key tiles are numbered across its pages (page p holds tiles
    // [cstart[p], cstart[p+1])) and group c of NG takes tiles c, c + NG, c + 2 NG, ... - all workgroups stream through
    // one narrow window of the cache instead of NG far-apart chunks, which the DRAM serves faster. Items group-major, pairs
    // fastest; XCD x (= blockIdx % 8 in dispatch order) takes the contiguous item range [x*T8, (x+1)*T8), so the pairs of
    // one tile - neighbours in the same key rows - share an L2.
    const uint32_t bid = blockIdx.x, xcd = bid % 8, local = bid / 8;
    const uint32_t t8 = (a.n_items + 7) / 8;
    const uint32_t w = xcd * t8 + local;
    if (local >= t8 || w >= a.n_items) return;
    const uint32_t npair = a.nkv / 2;
    const uint32_t pr = w % npair, c = w / npair;
    const uint32_t NG = a.n_chunks, T = a.cstart[a.n_pages];
    const uint32_t rs = a.rs;

    const int tid = threadIdx.x, lane = tid % 64;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);      // uniform: the tile loop is a scalar loop
    const int hd = wave;                                             // this wave's head in the pair; it loads K (0) or V (1)
    const uint32_t h = 2 * pr + hd;
    const int g = lane >> 4, n = lane & 15, hh = g & 1;
    const int kap = 16 * (g >> 1) + n;                               // this lane's key in the tile

    char * raw = smem;                                               // [2][32 keys][SL]
    char * wl = smem + RAW + wave * DEC_WLDS;
    uint8_t * Vs = (uint8_t *) wl;                                   // [32 keys][DEC_VST] int8 V, block-aligned
    char * Pl = wl + 32 * DEC_VST;                                   // [NKB][32 keys][8 rows] fp16 P'
    char * Qt = Pl + DEC_NKB * DEC_PBLK;                             // [NKB][DEC_QBLK] int8 query operands
    float * Ct = (float *) (Qt + DEC_NKB * DEC_QBLK);                // [NKB][8] scales, then [NKB][8] q4_0 starts

    // ---- tile loads: wave 0 loads K, wave 1 V, as buffer loads from a per-tile scalar base (the tile's first row of
    // the pair slice) whose range ends with the page: chunk q = 64 i + lane is key q / NCH, bytes 16 * (q % NCH) of the
    // slice; rows past the page's end, and lanes past the tile's chunks, read zeros (range check, no memory access)
    uint32_t vo[CPL];
    #pragma unroll
    for (int i = 0; i < CPL; i++) {
        const int q = 64 * i + lane;
        vo[i] = q < TCH ? (uint32_t) (q / G::NCH) * rs + 16u * (uint32_t) (q % G::NCH) : 0x80000000u;
    }
    // the page of tile tau, its first tile and its key count: by shift for uniform pages (a.ptl < 32), else by a walk of
    // the page table (pages only advance); the scalar loads of the walk wait for the LDS operations in flight too
    const uint32_t ptl = a.ptl, np1 = a.n_pages - 1;
    const uint32_t last_keys = a.pstart[a.n_pages] - a.pstart[np1];
    auto page_of = [&](uint32_t tau, uint32_t & pg) {
        if (ptl < 32u) pg = min(tau >> ptl, np1);
        else while (a.cstart[pg + 1] <= tau) pg++;
    };
    auto page_tile0 = [&](uint32_t pg) { return ptl < 32u ? pg << ptl : a.cstart[pg]; };
    auto page_keys = [&](uint32_t pg) { return ptl < 32u ? (pg < np1 ? 32u << ptl : last_keys) : a.pstart[pg + 1] - a.pstart[pg]; };
    auto tile_load = [&](pa_u4 (&X)[CPL], uint32_t pg, uint32_t j0, uint32_t nrec) {   // rows j0 .. of page pg
        const uint8_t * tb = (hd ? a.vp[pg] : a.kp[pg]) + (size_t) pr * G::SL + (size_t) j0 * rs;
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc((void *) tb, (short) 0, (int) nrec, 0x00020000);
        #pragma unroll
        for (int i = 0; i < CPL; i++) X[i] = __builtin_bit_cast(pa_u4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, vo[i], 0, 0));
    };
    auto tile_store = [&](const pa_u4 (&X)[CPL]) {
        char * dst = raw + hd * TCH * 16 + 16 * lane;
        #pragma unroll
        for (int i = 0; i < CPL; i++)
            if (i < CPL - 1 || 64 * (CPL - 1) + lane < TCH) *(pa_u4 *) (dst + 16 * 64 * i) = X[i];
    };

    // ---- the query rows' loads first, then the first two tiles' loads, so that the query preparation waits only for
    // its own loads (memory counters are in order). Each lane takes one (row, block, half): lane 8 r + 2 b + e holds
    // elements 32 b + 16 e .. +15 of row r (row 0 when past the rows, then zeroed), so every query value is quantized
    // once, and the two halves of a block sit in neighbouring lanes.
    const int qrl = lane >> 3, qbl = (lane >> 1) & 3, qhl = lane & 1;
    const bool qlive = qrl < (int) a.rows;
    const uint32_t qmask = qlive ? 0xffffffffu : 0u;
    pa_f4 qx[4];
    {
        const float * qp = a.q + ((size_t) h * a.rows + (qlive ? qrl : 0)) * DEC_HD + 32 * qbl + 16 * qhl;
        #pragma unroll
        for (int j = 0; j < 4; j++) qx[j] = *(const pa_f4 *) (qp + 4 * j);
    }
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t ntiles = (T - c + NG - 1) / NG;                   // >= 1: c < NG <= T
    uint32_t pl = 0, pc = 0;                                         // pages of the next tile to load / to compute
    auto load_tile = [&](pa_u4 (&X)[CPL], uint32_t tau) {            // tile tau, or (past the end) an empty range
        if (tau < T) {
            page_of(tau, pl);
            const uint32_t j0 = 32 * (tau - page_tile0(pl));
            // the range covers the tile's rows only (at most 32 of rs bytes, rs < 2^26 by the host's check), so a page
            // of any size keeps the 32-bit byte count exact; the pair's slice ends inside each row (nkv * hb <= rs)
            tile_load(X, pl, j0, min(page_keys(pl) - j0, 32u) * rs - pr * G::SL);
        } else {
            tile_load(X, pl, 0, 0u);
        }
    };
    // DEC_PF register sets: tile c + k NG in set k % DEC_PF, each set's batch issued strictly after the previous
    // set's (in-order counters: the wait before a tile covers only its own batch)
    pa_u4 X0[CPL], X1[CPL], X2[CPL];
    load_tile(X0, c);
    __builtin_amdgcn_sched_barrier(0);
    load_tile(X1, c + NG);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (DEC_PF == 3) load_tile(X2, c + 2 * NG);
    __builtin_amdgcn_sched_barrier(0);

    // ---- query rows: ggml's q8_0 of each 32-block (d = amax/127, id = 1/d, q = roundf(x*id), d -> fp16;
    // quantize_row_q8_0_ref), kept in the wave's LDS table [block][row][half][16 bytes] + a zero slot and read per tile
    // as the int8 A operand: lane (g, n) takes row slot n (row n % 8; slots 8-15 face keys 16-31), bytes 16*(g%2) .. +15
    // of the block, or the zero slot unless g / 2 == n / 8. Beside it: the fp16 query scale * s_mul per (block, row), and
    // for q4_0 K the MFMA accumulator start -8 * (sum of the row's block quants).
    {
        #pragma clang fp contract(off)
        float x[16];
        #pragma unroll
        for (int j = 0; j < 4; j++) {                                // a dead row is zeroed by a mask, so that the loads
            // stay where they were issued (whole vectors are bit-cast: clang's bit_cast of one ext-vector element reads
            // element 0)
            const pa_f4 v = __builtin_bit_cast(pa_f4, __builtin_bit_cast(pa_u4, qx[j]) & qmask);
            x[4 * j] = v[0]; x[4 * j + 1] = v[1]; x[4 * j + 2] = v[2]; x[4 * j + 3] = v[3];
        }
        float am = 0.0f;
        #pragma unroll
        for (int j = 0; j < 16; j++) am = fmaxf(am, fabsf(x[j]));
        am = fmaxf(am, dec_dpp<0xb1>(am));                           // the other half of the block: lane ^ 1
        const float d = am / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t wq[4] = {0, 0, 0, 0};
        int qsum = 0;
        #pragma unroll
        for (int j = 0; j < 16; j++) {
            const float t = x[j] * id;
            const int q = (int) roundf(t);
            qsum += q;
            wq[j / 4] |= ((uint32_t) q & 0xffu) << (8 * (j % 4));
        }
        qsum += __builtin_amdgcn_update_dpp(0, qsum, 0xb1, 0xf, 0xf, false);
        *(pa_u4 *) (Qt + qbl * DEC_QBLK + qrl * 32 + qhl * 16) = (pa_u4){wq[0], wq[1], wq[2], wq[3]};
        if (qhl == 0) {
            Ct[qbl * 8 + qrl] = (float) (_Float16) d * a.s_mul;
            Ct[DEC_NKB * 8 + qbl * 8 + qrl] = __builtin_bit_cast(float, -8 * qsum);
        }
        if (lane < DEC_NKB) *(pa_u4 *) (Qt + lane * DEC_QBLK + 256) = (pa_u4){0u, 0u, 0u, 0u};
        dec_wave_sync();
    }
    const int qoffa = (g >> 1) == (n >> 3) ? (n & 7) * 32 + hh * 16 : 256;   // this lane's A operand in a block table

    // ---- running state: O^T accumulators (lane (g, n): dims 16db + 4g + i, row slot n), per score-layout row i
    // (row 4*hh + i): reference max, exact max relative to it, sum
    pa_f4 O[DEC_ND];
    #pragma unroll
    for (int d = 0; d < DEC_ND; d++) O[d] = (pa_f4){0.f, 0.f, 0.f, 0.f};
    float mref[4], nm[4], mxr[4], lsum[4];
    #pragma unroll
    for (int i = 0; i < 4; i++) { mref[i] = -INFINITY; nm[i] = 0.0f; mxr[i] = -INFINITY; lsum[i] = 0.0f; }
    const _Float16 cb = FMT == 1 ? (_Float16) (-128.0f / 16777216.0f) : (_Float16) (-136.0f / 16777216.0f);
    const pa_h8 cneg = {cb, cb, cb, cb, cb, cb, cb, cb};
    float * arow = (float *) Pl;                                     // rescale factors by row (rare path scratch)
    const char * krow = raw + kap * G::SL, * vrow = raw + TCH * 16 + kap * G::SL;
    uint8_t * vdst = Vs + kap * DEC_VST;

    auto tile = [&](pa_u4 (&X)[CPL], uint32_t tau) {
        // ---- the tile's raw pair slices -> LDS (this wave's tensor), then this register set's next tile (DEC_PF steps
        // ahead; past the last one an empty range that loads nothing)
        page_of(tau, pc);
        const int nvalid = (int) min(32u, page_keys(pc) - 32 * (tau - page_tile0(pc)));
        dec_lds_barrier();                                           // both waves are done reading the previous tile
        tile_store(X);
        load_tile(X, tau + DEC_PF * NG);
        dec_lds_barrier();                                           // the tile's raw bytes are visible
        __builtin_amdgcn_sched_barrier(0);

        // ---- this lane's key: K operands and scales, V scales; V quants -> the aligned tile. The head's offset in the
        // pair slice (0 or HB) fixes every alignment at compile time; the branch is uniform.
        dec_v4i kq[DEC_NKB];
        float dkf[DEC_NKB];
        pa_h2 dvh[DEC_NKB];
        if (hd) dec_unpack<FMT, G::HB>(krow, vrow, vdst, hh, kq, dkf, dvh);
        else dec_unpack<FMT, 0>(krow, vrow, vdst, hh, kq, dkf, dvh);
        dec_wave_sync();
        __builtin_amdgcn_sched_barrier(0);

        // ---- S = Q K^T block by block on the int8 matrix cores
        dec_v4i T[DEC_NKB];
        #pragma unroll
        for (int b = 0; b < DEC_NKB; b++) {
            dec_v4i kb4 = kq[b];
            if constexpr (FMT == 2) {
                const int sh = 4 * hh;
                kb4 = (dec_v4i){(int) (((uint32_t) kb4.x >> sh) & 0x0f0f0f0fu), (int) (((uint32_t) kb4.y >> sh) & 0x0f0f0f0fu),
                                (int) (((uint32_t) kb4.z >> sh) & 0x0f0f0f0fu), (int) (((uint32_t) kb4.w >> sh) & 0x0f0f0f0fu)};
            }
            const dec_v4i qa = *(const dec_v4i *) (Qt + b * DEC_QBLK + qoffa);
            const dec_v4i qc = FMT == 2 ? *(const dec_v4i *) (Ct + DEC_NKB * 8 + b * 8 + 4 * hh) : (dec_v4i){0, 0, 0, 0};
            T[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa, kb4, qc, 0, 0, 0);
        }

        // ---- base-2 scores relative to the reference max: S = -mref + sum_b (dot_b * dq_b * s_mul) * dk_b
        float S[4] = {nm[0], nm[1], nm[2], nm[3]};
        #pragma unroll
        for (int b = 0; b < DEC_NKB; b++) {
            const pa_f4 cq = *(const pa_f4 *) (Ct + b * 8 + 4 * hh);   // query scale * s_mul, rows 4*hh + i
            #pragma unroll
            for (int i = 0; i < 4; i++) S[i] = fmaf((float) T[b][i] * cq[i], dkf[b], S[i]);
        }
        #pragma unroll
        for (int i = 0; i < 4; i++) S[i] = kap < nvalid ? S[i] : -INFINITY;
        const float smax = fmaxf(fmaxf(S[0], S[1]), fmaxf(S[2], S[3]));
        if (__any(smax > PMAX_LOG2 || mref[0] == -INFINITY)) {
            // rare: move the reference max of every row to its running max (uniform branch)
            #pragma unroll
            for (int i = 0; i < 4; i++) {
                const float rm = dec_rowmax32(S[i] - nm[i]);        // this tile's row max, absolute
                const float mn = fmaxf(mref[i], rm);
                const float alpha = mref[i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mref[i] - mn);
                const float nmn = mn == -INFINITY ? 0.0f : -mn;
                const float dlt = nmn - nm[i];
                S[i] += dlt;
                mxr[i] += dlt;
                lsum[i] *= alpha;
                mref[i] = mn;
                nm[i] = nmn;
                if (n == 0 && g < 2) arow[4 * g + i] = alpha;
            }
            dec_wave_sync();
            const float al = arow[n & 7];
            #pragma unroll
            for (int d = 0; d < DEC_ND; d++) O[d] *= al;
            dec_wave_sync();
        }
        float pr4[4];
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            mxr[i] = fmaxf(mxr[i], S[i]);
            pr4[i] = __builtin_amdgcn_exp2f(S[i]);
            lsum[i] += pr4[i];
        }
        const pa_h2 p01 = {(_Float16) pr4[0], (_Float16) pr4[1]}, p23 = {(_Float16) pr4[2], (_Float16) pr4[3]};
        // ---- P' = P * d_v per V block -> LDS [block][key][row], then back transposed as the PV B operand
        #pragma unroll
        for (int b = 0; b < DEC_NKB; b++) {
            const pa_u2 val = {pa_as_u32(p01 * dvh[b]), pa_as_u32(p23 * dvh[b])};
            *(pa_u2 *) (Pl + b * DEC_PBLK + kap * 16 + 8 * hh) = val;
        }
        dec_wave_sync();
        // ---- O^T += V^T P'^T per V block: P'^T by transposing 16-bit reads; V^T from the aligned tile by transposing
        // byte reads, int8 -> fp16 subnormal (q + 128) * 2^-24
        #pragma unroll
        for (int b = 0; b < DEC_NKB; b++) {
            __builtin_amdgcn_sched_barrier(0);
            const char * base = Pl + b * DEC_PBLK + (n & 1) * 8;
            const dec_h4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4f16((DEC_LDS dec_h4 *) (base + (8 * g + (n >> 2)) * 16));
            const dec_h4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4f16((DEC_LDS dec_h4 *) (base + (8 * g + 4 + (n >> 2)) * 16));
            const pa_h4 y0 = __builtin_bit_cast(pa_h4, x0), y1 = __builtin_bit_cast(pa_h4, x1);
            const pa_h8 pb = {y0[0], y0[1], y0[2], y0[3], y1[0], y1[1], y1[2], y1[3]};
            #pragma unroll
            for (int db = 2 * b; db < 2 * b + 2; db++) {
                const dec_v2i rv = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                    (DEC_LDS dec_v2i *) (Vs + (8 * g + (n >> 1)) * DEC_VST + 16 * db + 8 * (n & 1)));
                const uint32_t x0 = (uint32_t) rv.x ^ 0x80808080u, x1 = (uint32_t) rv.y ^ 0x80808080u;
                const pa_u4 u = {pa_perm(x0, x0, 0x0c010c00u), pa_perm(x0, x0, 0x0c030c02u), pa_perm(x1, x1, 0x0c010c00u),
                                 pa_perm(x1, x1, 0x0c030c02u)};
                const pa_h8 va = __builtin_bit_cast(pa_h8, u);
                O[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb, O[db], 0, 0, 0);
                O[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cneg, pb, O[db], 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        dec_wave_sync();
    };
    // groups of DEC_PF tiles, then the rest: no exit inside a group, so the load order (X0's batch, X1's, ...) is the
    // same on every path into a tile and the wait before each tile covers only its own batch
    uint32_t tau = c;
    uint32_t t = 0;
    for (; t + DEC_PF <= ntiles; t += DEC_PF) {
        tile(X0, tau);
        tile(X1, tau + NG);
        if constexpr (DEC_PF == 3) tile(X2, tau + 2 * NG);
        tau += DEC_PF * NG;
    }
    if (t < ntiles) tile(X0, tau);
    if (t + 1 < ntiles) tile(X1, tau + NG);

    // ---- this wave's head: rows' (sum, exact max) over the lanes; O rebased from the reference max to the exact one
    // and written from lanes n < 8 (final result for a single group, else the group's split-K slot)
    float lt4[4], mt4[4], f4[4];
    #pragma unroll
    for (int i = 0; i < 4; i++) {
        lt4[i] = dec_rowsum32(lsum[i]);
        mt4[i] = dec_rowmax32(mxr[i]) - nm[i];                     // the exact max (base 2); -inf without keys
        f4[i] = mref[i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mref[i] - mt4[i]);
        if (n == 0 && g < 2) {                                       // row 4*hh + i: the factor for the O lanes
            arow[4 * g + i] = f4[i] * 16777216.0f;                   // (the accumulator holds O * 2^-24)
            arow[8 + 4 * g + i] = mt4[i];
            arow[16 + 4 * g + i] = lt4[i] * f4[i];
        }
    }
    dec_wave_sync();
    const bool direct = a.fused;                                     // one group holds the call: the final result
    const uint32_t r = n & 7;
    if (n < 8 && r < a.rows) {
        const float fo = arow[r], M = arow[8 + r], L = arow[16 + r];
        #pragma unroll
        for (int d = 0; d < DEC_ND; d++) {
            const pa_f4 v = O[d] * fo;
            if (direct) *(pa_f4 *) (a.O + ((size_t) h * a.rows + r) * DEC_HD + 16 * d + 4 * g) = v;
            else *(pa_f4 *) (a.po + (((size_t) h * a.qr + r) * a.slots + a.slot0 + c) * DEC_HD + 16 * d + 4 * g) = v;
        }
        if (g == 0) {
            if (direct) { a.m[(size_t) h * a.rows + r] = M == -INFINITY ? -INFINITY : M * PA_LN2; a.l[(size_t) h * a.rows + r] = L; }
            else a.pml[((size_t) h * a.qr + r) * a.slots + a.slot0 + c] = make_float2(M, L);
        }
    }
}

hipError_t launch_decode(int fmt, const AttnArgs & a, uint32_t grid, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    // the events (optional) are recorded by the launch itself at the kernel's start and end
    if (fmt == 1) hipExtLaunchKernelGGL((dec_kernel<1>), dim3(grid), dim3(128), 0, st, ev0, ev1, 0, a);
    else if (fmt == 2) hipExtLaunchKernelGGL((dec_kernel<2>), dim3(grid), dim3(128), 0, st, ev0, ev1, 0, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace pa_hip
