// pa_decode.hip - decode partial attention for up to 8 query rows per KV head (one token x GQA 8), q8_0 / q4_0 K and V,
// ggml query rounding, head_dim 128 (gfx950).
//
// One workgroup = one pair of KV heads x one chunk of keys inside one page, 2*TPR waves: wave w computes head w % 2 of
// tile w / 2 of every round (a round = TPR tiles of 32 keys). HBM traffic is fully coalesced: per round the workgroup
// reads the pair's contiguous slice of every key row (2 x 136 bytes for q8_0) of K and V with 16-byte loads, lane by
// lane along the rows (K by the first half of the waves, V by the second), two rounds ahead in registers. A round's
// bytes are written raw into LDS; each wave then reads its head's K quants from there as the MFMA operand (unaligned
// 16-byte LDS reads), and copies its V quants into its own block-aligned tile for the transposing reads.
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

template <int FMT> struct DecGeom {
    static constexpr int BB = FMT == 1 ? 34 : 18;          // bytes per quant block
    static constexpr int HB = BB * DEC_NKB;                // bytes per head in a key row (136 / 72)
    static constexpr int SL = 2 * HB;                      // a head pair's slice of a key row (272 / 144)
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
// workgroup barrier that orders LDS only: the vector-memory loads in flight (the next rounds) are not waited for
__device__ __forceinline__ void dec_lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// 16 bytes at byte offset S (compile-time) past a 16-byte aligned LDS address, from naturally aligned dword reads and
// byte alignment: unaligned LDS reads run at a fraction of the aligned rate
template <int S> __device__ __forceinline__ pa_u4 dec_lds16(const char * base16) {
    const uint32_t * p = (const uint32_t *) __builtin_assume_aligned(base16, 16);
    constexpr int W = S / 4, B = S % 4;
    uint32_t d[5];
    #pragma unroll
    for (int k = 0; k < (B ? 5 : 4); k++) d[k] = p[W + k];
    pa_u4 r;
    #pragma unroll
    for (int j = 0; j < 4; j++) r[j] = B ? __builtin_amdgcn_alignbyte(d[j + 1], d[j], B) : d[j];
    return r;
}

// this lane's K operands (16 quant bytes of each block; q8_0: half hh) and block scales from a raw key row (16-byte
// aligned) of the round, for the head at slice offset HD * HB
template <int FMT, int HD>
__device__ __forceinline__ void dec_k_ops(const char * krow, int hh, dec_v4i (&kq)[DEC_NKB], float (&dkf)[DEC_NKB]) {
    using G = DecGeom<FMT>;
    #pragma unroll
    for (int b = 0; b < DEC_NKB; b++) {
        const int o = HD * G::HB + G::BB * b + 2;                    // quants of block b (compile-time after unrolling)
        const char * base = krow + (o & ~15) + (FMT == 1 ? 16 * hh : 0);
        switch (o & 15) {                                            // resolved at compile time
            case 0: kq[b] = __builtin_bit_cast(dec_v4i, dec_lds16<0>(base)); break;
            case 2: kq[b] = __builtin_bit_cast(dec_v4i, dec_lds16<2>(base)); break;
            case 4: kq[b] = __builtin_bit_cast(dec_v4i, dec_lds16<4>(base)); break;
            case 6: kq[b] = __builtin_bit_cast(dec_v4i, dec_lds16<6>(base)); break;
            case 8: kq[b] = __builtin_bit_cast(dec_v4i, dec_lds16<8>(base)); break;
            case 10: kq[b] = __builtin_bit_cast(dec_v4i, dec_lds16<10>(base)); break;
            case 12: kq[b] = __builtin_bit_cast(dec_v4i, dec_lds16<12>(base)); break;
            default: kq[b] = __builtin_bit_cast(dec_v4i, dec_lds16<14>(base)); break;
        }
        dkf[b] = pa_f16_bits_to_f32(*(const uint16_t *) (krow + HD * G::HB + G::BB * b));
    }
}

// V blocks of the wave's 32 keys from the raw round into the aligned tile [key][32 * block] (q4_0: nibbles unpacked to
// bytes, element order), lane l: key l / 2, half l % 2. q8_0 block 3 is 8-byte aligned in the raw rows already and is
// read from there.
template <int FMT, int HD>
__device__ __forceinline__ void dec_v_repack(const char * vtile, uint8_t * Vs, int lane) {
    using G = DecGeom<FMT>;
    const int key = lane >> 1, half = lane & 1;
    const char * vrow = vtile + key * G::SL;
    #pragma unroll
    for (int b = 0; b < (FMT == 1 ? DEC_NKB - 1 : DEC_NKB); b++) {
        const int o = HD * G::HB + G::BB * b + 2;
        const char * base = vrow + (o & ~15) + (FMT == 1 ? 16 * half : 0);
        pa_u4 x;
        switch (o & 15) {
            case 0: x = dec_lds16<0>(base); break;
            case 2: x = dec_lds16<2>(base); break;
            case 4: x = dec_lds16<4>(base); break;
            case 6: x = dec_lds16<6>(base); break;
            case 8: x = dec_lds16<8>(base); break;
            case 10: x = dec_lds16<10>(base); break;
            case 12: x = dec_lds16<12>(base); break;
            default: x = dec_lds16<14>(base); break;
        }
        if constexpr (FMT == 2) {
            const int sh = 4 * half;
            x = (pa_u4){(x.x >> sh) & 0x0f0f0f0fu, (x.y >> sh) & 0x0f0f0f0fu, (x.z >> sh) & 0x0f0f0f0fu, (x.w >> sh) & 0x0f0f0f0fu};
        }
        *(pa_u4 *) (Vs + key * DEC_VST + 32 * b + 16 * half) = x;
    }
}

template <int FMT, int TPR>
__global__ __launch_bounds__(128 * TPR, 2) void dec_kernel(const AttnArgs a) {
    using G = DecGeom<FMT>;
    constexpr int NW = 2 * TPR;                                      // waves
    constexpr int RK = 32 * TPR;                                     // keys per round
    constexpr int TCH = RK * G::NCH;                                 // chunks per tensor per round
    constexpr int LPT = 64 * NW / 2;                                 // lanes loading one tensor
    constexpr int CPL = (TCH + LPT - 1) / LPT;                       // chunks per lane per round
    constexpr int RAW = 2 * TCH * 16;                                // raw round bytes in LDS: K rows, then V rows
    constexpr int COMB = NW * 8 * DEC_HD * 4 + NW * 8 * 16;         // end: per-wave O rows + (mref, mtrue, l)
    constexpr int MAIN = RAW + NW * DEC_WLDS;
    constexpr int LDS = MAIN > COMB ? MAIN : COMB;
    __shared__ __attribute__((aligned(16))) char smem[LDS];

    // ---- which (chunk, head pair): items chunk-major, pairs fastest; XCD x (= blockIdx % 8 in dispatch order) takes
    // the contiguous item range [x*T8, (x+1)*T8), so the pairs of one chunk - neighbours in the same key rows - share an L2
    const uint32_t bid = blockIdx.x, xcd = bid % 8, local = bid / 8;
    const uint32_t t8 = (a.n_items + 7) / 8;
    const uint32_t w = xcd * t8 + local;
    if (local >= t8 || w >= a.n_items) return;
    const uint32_t npair = a.nkv / 2;
    const uint32_t pr = w % npair, c = w / npair;
    uint32_t p = 0;
    while (a.cstart[p + 1] <= c) p++;                                // the page holding chunk c
    const uint32_t k0 = (c - a.cstart[p]) * a.chunk;
    const uint32_t k1 = min(k0 + a.chunk, a.pstart[p + 1] - a.pstart[p]);
    const uint32_t rs = a.rs;

    const int tid = threadIdx.x, lane = tid % 64;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);      // uniform: the round loop is a scalar loop
    const int hd = wave & 1, ts = wave >> 1;                         // this wave's head in the pair, tile in the round
    const uint32_t h = 2 * pr + hd;
    const int g = lane >> 4, n = lane & 15, hh = g & 1;
    const int kap = 16 * (g >> 1) + n;                               // this lane's key in the tile

    char * raw = smem;                                               // [2][RK keys][SL]: the round's K, V slices
    char * wl = smem + RAW + wave * DEC_WLDS;
    uint8_t * Vs = (uint8_t *) wl;                                   // [32 keys][DEC_VST] int8 V, block-aligned
    char * Pl = wl + 32 * DEC_VST;                                   // [NKB][32 keys][8 rows] fp16 P'
    char * Qt = Pl + DEC_NKB * DEC_PBLK;                             // [NKB][DEC_QBLK] int8 query operands
    float * Ct = (float *) (Qt + DEC_NKB * DEC_QBLK);                // [NKB][8] scales, then [NKB][8] q4_0 starts

    // ---- load roles: the first NW/2 waves load K, the rest V; chunk q = i*LPT + lt of the tensor's round is key q / NCH,
    // bytes 16 * (q % NCH) of the pair slice
    const bool ldv = wave >= NW / 2;
    const int lt = tid - (ldv ? 64 * NW / 2 : 0);
    const uint8_t * tbase = (ldv ? a.vp[p] : a.kp[p]) + (size_t) pr * G::SL;
    uint32_t qkey[CPL], qoff[CPL];
    #pragma unroll
    for (int i = 0; i < CPL; i++) {
        const int q = min(i * LPT + lt, TCH - 1);                    // a lane past the round's chunks reloads the last
        qkey[i] = (uint32_t) (q / G::NCH);
        qoff[i] = 16u * (uint32_t) (q % G::NCH);
    }
    auto round_load = [&](pa_u4 (&X)[CPL], uint32_t jr) {
        const uint32_t last = k1 - 1 - jr;                           // the round's last valid key (rows past it reload it)
        #pragma unroll
        for (int i = 0; i < CPL; i++) {
            const uint32_t row = jr + min(qkey[i], last);
            X[i] = pa_ld<pa_u4>(tbase + (size_t) row * rs + qoff[i]);
        }
    };
    auto round_store = [&](const pa_u4 (&X)[CPL]) {
        char * dst = raw + (ldv ? TCH * 16 : 0) + 16 * lt;
        #pragma unroll
        for (int i = 0; i < CPL; i++)
            if (i < CPL - 1 || (CPL - 1) * LPT + lt < TCH) *(pa_u4 *) (dst + 16 * i * LPT) = X[i];
    };

    // ---- the query rows' loads first, then the first two rounds' loads, so that the query preparation waits only for
    // its own loads (memory counters are in order). Lane (g, n): row n % 8 (row 0 when past the rows, then zeroed),
    // elements 16*(g%2) .. +15 of every block.
    const int qr8 = n & 7;
    const bool qlive = qr8 < (int) a.rows;
    pa_f4 qx[DEC_NKB][4];
    {
        const float * qrow = a.q + ((size_t) h * a.rows + (qlive ? qr8 : 0)) * DEC_HD + 16 * hh;
        #pragma unroll
        for (int b = 0; b < DEC_NKB; b++)
            #pragma unroll
            for (int j = 0; j < 4; j++) qx[b][j] = *(const pa_f4 *) (qrow + 32 * b + 4 * j);
    }
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t nround = (k1 - k0 + RK - 1) / RK;                 // >= 1: the chunk is not empty
    pa_u4 X0[CPL], X1[CPL];                                          // rounds 0, 2, 4, ... and 1, 3, 5, ...
    round_load(X0, k0);
    __builtin_amdgcn_sched_barrier(0);                               // X0's loads strictly before X1's (in-order counts)
    round_load(X1, nround > 1 ? k0 + RK : k0);
    __builtin_amdgcn_sched_barrier(0);

    // ---- query rows: ggml's q8_0 of each 32-block (d = amax/127, id = 1/d, q = roundf(x*id), d -> fp16;
    // quantize_row_q8_0_ref), kept in the wave's LDS table and read per tile as the int8 A operand: lane (g, n) takes
    // row slot n (row n % 8; slots 8-15 face keys 16-31), bytes 16*(g%2) .. +15 of the block, or the zero slot unless
    // g / 2 == n / 8. Beside it: the fp16 query scale * s_mul per (block, row), and for q4_0 K the MFMA accumulator start
    // -8 * (sum of the row's block quants).
    {
        #pragma clang fp contract(off)
        #pragma unroll
        for (int b = 0; b < DEC_NKB; b++) {
            float x[16];
            #pragma unroll
            for (int j = 0; j < 4; j++) {
                const pa_f4 v = qlive ? qx[b][j] : (pa_f4){0.f, 0.f, 0.f, 0.f};
                x[4 * j] = v[0]; x[4 * j + 1] = v[1]; x[4 * j + 2] = v[2]; x[4 * j + 3] = v[3];
            }
            float am = 0.0f;
            #pragma unroll
            for (int j = 0; j < 16; j++) am = fmaxf(am, fabsf(x[j]));
            am = fmaxf(am, __shfl_xor(am, 16));                      // the other half of the block: lane ^ 16
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
            qsum += __shfl_xor(qsum, 16);
            if (g < 2 && n < 8) {                                    // (row n, half g) for every block
                *(pa_u4 *) (Qt + b * DEC_QBLK + n * 32 + g * 16) = (pa_u4){wq[0], wq[1], wq[2], wq[3]};
                if (g == 0) {
                    Ct[b * 8 + n] = (float) (_Float16) d * a.s_mul;
                    Ct[DEC_NKB * 8 + b * 8 + n] = __builtin_bit_cast(float, -8 * qsum);
                }
            }
            if (lane == 0) *(pa_u4 *) (Qt + b * DEC_QBLK + 256) = (pa_u4){0u, 0u, 0u, 0u};
        }
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

    // this wave's tile in the raw round: this lane's K and V key rows (pair slices, 16-byte aligned), the V rows
    const char * krow = raw + (32 * ts + kap) * G::SL;
    const char * vrow = krow + TCH * 16;
    const char * vtile = raw + TCH * 16 + 32 * ts * G::SL;

    uint32_t jr = k0;
    auto round = [&](pa_u4 (&X)[CPL]) {
        dec_lds_barrier();                                           // every wave is done reading the previous round
        round_store(X);
        {   // this register set's next round (two rounds ahead; past the chunk's end it reloads the last rows)
            const uint32_t jn = jr + 2 * RK < k1 ? jr + 2 * RK : jr;
            round_load(X, jn);
        }
        dec_lds_barrier();                                           // the round's raw bytes are visible
        const uint32_t jt = jr + 32 * ts;
        const int nvalid = jt < k1 ? (int) min(32u, k1 - jt) : 0;
        if (nvalid == 0) return;                                     // uniform: this wave's tile is past the chunk
        __builtin_amdgcn_sched_barrier(0);

        // ---- from the raw round: this lane's K operands and scales, V scales; the V quants -> the wave's aligned tile.
        // Byte offsets of the head inside the pair slice differ by 8 (mod 16), so each head has its own (compile-time)
        // alignment; the branch is uniform.
        dec_v4i kq[DEC_NKB];
        float dkf[DEC_NKB];
        pa_h2 dvh[DEC_NKB];
        if (hd == 0) { dec_k_ops<FMT, 0>(krow, hh, kq, dkf); dec_v_repack<FMT, 0>(vtile, Vs, lane); }
        else { dec_k_ops<FMT, 1>(krow, hh, kq, dkf); dec_v_repack<FMT, 1>(vtile, Vs, lane); }
        #pragma unroll
        for (int b = 0; b < DEC_NKB; b++) {
            const _Float16 dv = __builtin_bit_cast(_Float16, *(const uint16_t *) (vrow + hd * G::HB + G::BB * b));
            dvh[b] = (pa_h2){dv, dv};
        }
        dec_wave_sync();
        __builtin_amdgcn_sched_barrier(0);

        // ---- S = Q K^T block by block on the int8 matrix cores
        dec_v4i T[DEC_NKB];
        #pragma unroll
        for (int b = 0; b < DEC_NKB; b++) {
            dec_v4i kb = kq[b];
            if constexpr (FMT == 2) {
                const int sh = 4 * hh;
                kb = (dec_v4i){(int) (((uint32_t) kb.x >> sh) & 0x0f0f0f0fu), (int) (((uint32_t) kb.y >> sh) & 0x0f0f0f0fu),
                               (int) (((uint32_t) kb.z >> sh) & 0x0f0f0f0fu), (int) (((uint32_t) kb.w >> sh) & 0x0f0f0f0fu)};
            }
            const dec_v4i qa = *(const dec_v4i *) (Qt + b * DEC_QBLK + qoffa);
            const dec_v4i qc = FMT == 2 ? *(const dec_v4i *) (Ct + DEC_NKB * 8 + b * 8 + 4 * hh) : (dec_v4i){0, 0, 0, 0};
            T[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa, kb, qc, 0, 0, 0);
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
                const char * vsrc = (FMT == 1 && b == DEC_NKB - 1)
                    ? vtile + (8 * g + (n >> 1)) * G::SL + hd * G::HB + G::BB * b + 2 + 16 * (db & 1) + 8 * (n & 1)
                    : (const char *) Vs + (8 * g + (n >> 1)) * DEC_VST + 16 * db + 8 * (n & 1);
                const dec_v2i rv = __builtin_amdgcn_ds_read_tr8_b64_v2i32((DEC_LDS dec_v2i *) vsrc);
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
    // pairs of rounds, then an odd last one: no exit between the two halves, so the load order (X0's batch before X1's)
    // is the same on every path into a round and the wait before each round covers only its own batch
    for (uint32_t r = 0; r + 1 < nround; r += 2) {
        round(X0);
        jr += RK;
        round(X1);
        jr += RK;
    }
    if (nround & 1) round(X0);

    // ---- wave state -> LDS: O rows (lanes n < 8), (mref, exact max, sum) per row
    float lt4[4], mt[4];
    #pragma unroll
    for (int i = 0; i < 4; i++) {
        lt4[i] = dec_rowsum32(lsum[i]);
        mt[i] = dec_rowmax32(mxr[i]) - nm[i];                      // -inf for a wave without keys
    }
    __syncthreads();                                                 // every wave is done with its tiles
    float * cO = (float *) smem;                                     // [NW][8][HD]
    float * cS = cO + NW * 8 * DEC_HD;                               // [NW][8][4]: mref, mtrue, l
    if (n < 8) {
        #pragma unroll
        for (int d = 0; d < DEC_ND; d++) *(pa_f4 *) (cO + ((size_t) wave * 8 + n) * DEC_HD + 16 * d + 4 * g) = O[d];
    }
    if (n == 0 && g < 2) {
        #pragma unroll
        for (int i = 0; i < 4; i++) *(pa_f4 *) (cS + (wave * 8 + 4 * g + i) * 4) = (pa_f4){mref[i], mt[i], lt4[i], 0.0f};
    }
    __syncthreads();

    // ---- merge the waves of each head (waves hd, hd + 2, ...); write the final result (one chunk) or a split-K slot
    const bool direct = a.n_chunks == 1 && a.fused;
    const uint32_t nrows = min(a.rows, 8u);
    for (uint32_t e = tid; e < 2 * nrows * (DEC_HD / 4); e += 64 * NW) {
        const uint32_t eh = e / (nrows * (DEC_HD / 4)), er = e % (nrows * (DEC_HD / 4));
        const uint32_t r = er / (DEC_HD / 4), d4 = er % (DEC_HD / 4);
        const uint32_t hw = 2 * pr + eh;
        float M = -INFINITY;
        #pragma unroll
        for (int t = 0; t < TPR; t++) M = fmaxf(M, cS[((2 * t + eh) * 8 + r) * 4 + 1]);
        pa_f4 acc = {0.f, 0.f, 0.f, 0.f};
        float L = 0.0f;
        if (M != -INFINITY) {
            #pragma unroll
            for (int t = 0; t < TPR; t++) {
                const int q = 2 * t + eh;
                const pa_f4 st = *(const pa_f4 *) (cS + (q * 8 + r) * 4);
                const float wt = st[0] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(st[0] - M);
                L += wt * st[2];
                acc += (wt * 16777216.0f) * *(const pa_f4 *) (cO + ((size_t) q * 8 + r) * DEC_HD + 4 * d4);
            }
        }
        if (direct) {
            *(pa_f4 *) (a.O + ((size_t) hw * a.rows + r) * DEC_HD + 4 * d4) = acc;
            if (d4 == 0) { a.m[(size_t) hw * a.rows + r] = M == -INFINITY ? -INFINITY : M * PA_LN2; a.l[(size_t) hw * a.rows + r] = L; }
        } else {
            const size_t slot = a.slot0 + c;
            *(pa_f4 *) (a.po + ((slot * a.nkv + hw) * a.qr + r) * DEC_HD + 4 * d4) = acc;
            if (d4 == 0) a.pml[(slot * a.nkv + hw) * a.qr + r] = make_float2(M, L);
        }
    }
}

hipError_t launch_decode(int fmt, int tpr, const AttnArgs & a, uint32_t grid, hipStream_t st) {
    if (fmt == 1 && tpr == 1) hipLaunchKernelGGL((dec_kernel<1, 1>), dim3(grid), dim3(128), 0, st, a);
    else if (fmt == 1 && tpr == 2) hipLaunchKernelGGL((dec_kernel<1, 2>), dim3(grid), dim3(256), 0, st, a);
    else if (fmt == 2 && tpr == 1) hipLaunchKernelGGL((dec_kernel<2, 1>), dim3(grid), dim3(128), 0, st, a);
    else if (fmt == 2 && tpr == 2) hipLaunchKernelGGL((dec_kernel<2, 2>), dim3(grid), dim3(256), 0, st, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace pa_hip
