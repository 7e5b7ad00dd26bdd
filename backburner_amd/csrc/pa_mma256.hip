// pa_mma256.hip - partial attention at head dim 256, the reference's compile-time shape (phone-attn.h:78-79: 48 query
// rows = 8 tokens x GQA 6 per KV head), over q8_0 / q4_0 / f16 K and V on fp16 matrix cores (gfx950). Queries are
// f16(q*scale) (PA_QMODE_F16, the reference engines' Qs, phone-attn.h:595-599), or f16(q) for f16 K in
// PA_QMODE_GGML (ggml's f16 vec_dot type; the scale then multiplies the score). In PA_QMODE_GGML over quantized K
// (EX) the scores are ggml's exact integer block dots: K staged as its integer quants with the block scales beside the
// tile, Q as ggml's q8_0 quants times 2^-s_b; per 32-dim block one MFMA gives the integer dot and one more the
// product of the key's and the row's block scales (see mm_prep_q in pa_mma.hip for the scale pair), summed in fp32.
//
// One workgroup = one KV head x one block of 64 query rows x one chunk of consecutive 32-key tiles; 4 waves of 16 rows
// (48 rows: three waves compute, the fourth only stages). Per tile the workgroup dequantizes K and V once into LDS as
// fp16 (d*q rounded once, as the hd-128 kernel and the Metal engine's dequant, pa-metal.mm:60-66), double-buffered, the
// next tiles' raw bytes in flight in registers. Each computing wave then runs v_mfma_f32_16x16x32_f16:
//   S^T (16 keys x 16 rows) = K . Q'^T per 16-key half kh, over 8 steps of 32 dims (Q' stays in registers), so lane
//   (g, n) holds row n's scores of keys 16kh + 4g + i (i < 4);
//   O^T (16 dims x 16 rows) += V^T . P^T per dim block (16 blocks), one step over the tile's 32 keys taken in the order
//   the scores sit in (MFMA k index 8g + 4kh + i = key 16kh + 4g + i): the P operand is the lane's own 8 probabilities,
//   and V^T comes from two transposing reads (ds_read_b64_tr_b16) per dim block.
// A row's maximum and sum need the 4 lanes n, n + 16, n + 32, n + 48 (two lane swaps). Online softmax in base 2 with a
// reference max that moves only when a score exceeds it by more than 2^MM_PMAX (O is rescaled rarely); the exact max is
// tracked beside it. Output: one split-K slot per workgroup (O unnormalised against the base-2 max, max, sum) or the
// final (O, m, l) when the call has a single chunk.
//
// Reference roles: pa_attn + pa_merge of the Metal engine at this shape (pa-metal.mm:22-131: per (chunk, KV head) a
// threadgroup of 48 rows dequantizes 32-key K/V blocks into threadgroup memory as half, S = QK^T and O += PV on
// simdgroup matrices, online softmax, one slot per chunk), and sme_attn_partial's semantics (phone-attn.h:63-65).
#include "pa_mma.h"
#include <hip/hip_ext.h>

namespace pa_hip {

// LDS geometry per head dim: K row stride 2 HD + 16 B (528 B = 132 dwords at 256, 272 B = 68 at 128: 16 keys' 16-byte
// reads at one dim offset hit distinct banks), V row stride 2 HD + 64 B (576 / 320 B: a transposing read's 4 rows x
// 32 bytes hit distinct banks), and for EX the tile's K block scales [key][HD / 32 blocks] fp16. Two stages: 35,840 B
// each at head dim 256, 19,200 B at 128.
template <int HD> struct M2Geom {
    static constexpr int NBLK = HD / 32;                      // quant blocks per head row
    static constexpr int KST = 2 * HD + 16, VST = 2 * HD + 64;
    static constexpr int KT = 32 * KST, VT = 32 * VST, KSC = 32 * 2 * NBLK;
    static constexpr int STAGE = KT + VT + KSC;
};

// v_permlane16_swap of a value with itself gives every lane the values of lanes l & ~16 and l | 16
__device__ __forceinline__ float m2_max16(float v) {    // max over lanes l and l ^ 16
    const auto t = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v), false, false);
    return fmaxf(__builtin_bit_cast(float, (unsigned) t[0]), __builtin_bit_cast(float, (unsigned) t[1]));
}
__device__ __forceinline__ float m2_sum16(float v) {    // sum over lanes l and l ^ 16
    const auto t = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v), false, false);
    return __builtin_bit_cast(float, (unsigned) t[0]) + __builtin_bit_cast(float, (unsigned) t[1]);
}

// SKIP: waves whose 16 rows are all past the call's rows only stage (one row block narrower than 64 rows).
// EX: exact block dots in ggml's query rounding (quantized K only). WPS: waves per SIMD the registers are sized for.
// Instantiated at head dim 256; at 128 (three waves per SIMD, 167 VGPRs) the 16-row waves measured slower than the
// 32-row mma_kernel on verify (157 against 111 us), each wave reading the whole K / V^T tile from LDS.
template <int HD, int FMT, bool SKIP, bool EX, int WPS>
__global__ __launch_bounds__(256, WPS) void mma256_kernel(const AttnArgs a) {
    static_assert(!EX || FMT != 0, "exact block dots need quantized K");
    using G2 = M2Geom<HD>;
    constexpr int NBLK = G2::NBLK, M2_KST = G2::KST, M2_VST = G2::VST, M2_KT = G2::KT, M2_VT = G2::VT;
    constexpr int M2_STAGE = G2::STAGE;
    // NB tiles' raw bytes are in flight while a tile is computed (a ring of NB register buffers); 3 to 5 measured no
    // faster than 2 at 48 rows x 4 KV heads x 65k q8_0 keys
    constexpr int NT = 256, NB = 2;
    constexpr int UPT = 128 * NBLK / NT;                             // staging units per thread (128 NBLK per tile)
    __shared__ __attribute__((aligned(16))) char smem[2 * M2_STAGE];

    // ---- which (chunk, KV head, row block): row blocks fastest, consecutive items on one XCD (blockIdx % 8 in dispatch
    // order takes a contiguous item range), so the workgroups sharing a chunk's K/V share its L2
    const uint32_t bid = blockIdx.x, xcd = bid % 8, local = bid / 8;
    const uint32_t t8 = (a.n_items + 7) / 8;
    const uint32_t w = xcd * t8 + local;
    if (local >= t8 || w >= a.n_items) return;
    const uint32_t rb = w % a.nrb, h = (w / a.nrb) % a.nkv, c = w / (a.nrb * a.nkv);
    const uint32_t T = a.cstart[a.n_pages];
    const uint32_t t0 = c * a.chunk, ntiles = min(t0 + a.chunk, T) - t0;

    const int tid = threadIdx.x, lane = tid % 64;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const int g = lane >> 4, n = lane & 15;
    const uint32_t row = rb * 64 + 16 * wave + n;
    const bool rlive = row < a.rows;
    const bool wlive = !SKIP || rb * 64 + 16 * wave < a.rows;       // uniform: the wave has a live row

    MmCursor cl, cc;
    cl.init(a); cc.init(a);

    // ---- staging units: u = tid + 256 i -> tensor 4 i / NBLK (uniform), key (u / (2 NBLK)) & 31, block (u >> 1) &
    // (NBLK - 1), half u & 1
    using F = MmFmt<FMT>;
    MmRaw<FMT> R[NB][UPT];                                           // tile j's raw bytes in R[j % NB]
    auto load_tile = [&](MmRaw<FMT> (&Rb)[UPT], uint32_t tau, bool live) {
        if (live) cl.seek(a, tau);
        const uint32_t j0 = live ? 32 * (tau - cl.tb) : 0u;
        const uint32_t last = live ? cl.nk - 1 - j0 : 0u;
        const uint32_t nrec = live ? min(last + 1, 32u) * a.rs : 0u;   // the tile's rows only (rs < 2^26)
        #pragma unroll
        for (int i = 0; i < UPT; i++) {
            const int u = tid + NT * i;
            const int tensor = 4 * i / NBLK, key = (u / (2 * NBLK)) & 31, blk = (u >> 1) & (NBLK - 1), half = u & 1;
            const uint8_t * base = (tensor ? cl.vb : cl.kb) + (size_t) h * a.hb + (size_t) j0 * a.rs;
            const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc((void *) base, (short) 0, (int) nrec, 0x00020000);
            mm_load_unit_buf_al<FMT>(Rb[i], rsrc, min((uint32_t) key, last) * a.rs + blk * F::BB, half,
                                     (uint32_t) (uintptr_t) base);
        }
    };
    auto store_tile = [&](const MmRaw<FMT> (&Rb)[UPT], int stage) {
        char * st = smem + stage * M2_STAGE;
        #pragma unroll
        for (int i = 0; i < UPT; i++) {
            const int u = tid + NT * i;
            const int tensor = 4 * i / NBLK, key = (u / (2 * NBLK)) & 31, blk = (u >> 1) & (NBLK - 1), half = u & 1;
            pa_u4 lo, hi;
            if (EX && tensor == 0) {                                 // K: integer quants, the block scale beside the tile
                mm_dequant<FMT, true>(Rb[i], half, lo, hi);
                if (half == 0) *(uint16_t *) (st + M2_KT + M2_VT + 2 * NBLK * key + 2 * blk) = (uint16_t) Rb[i].d;
            } else {
                mm_dequant<FMT>(Rb[i], half, lo, hi);
            }
            char * dst = (tensor ? st + M2_KT + key * M2_VST : st + key * M2_KST) + 2 * (32 * blk + 16 * half);
            *(pa_u4 *) dst = lo;
            *(pa_u4 *) (dst + 16) = hi;
        }
    };

    #pragma unroll
    for (int i = 0; i < NB; i++) {
        load_tile(R[i], t0 + i, i == 0 || ntiles > (uint32_t) i);
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- Q' as the B operand: lane (g, n) holds row n, dims 32 s + 8 g .. +7. EX: per 32-dim block s, ggml's q8_0 quants
    // (quantize_row_q8_0_ref: d = amax / 127, q = roundf(x / d); the block's 32 values sit in lanes n, n + 16, n + 32,
    // n + 48) times 2^-s_b, exact in fp16, and in dqw[s] (lanes g = 0) the pair (hi, lo) summing to fp16(d) * scale *
    // log2 e * 2^s_b to about 22 bits, s_b putting it in [8, 16)
    mm_h8 Qf[NBLK];
    uint32_t dqw[NBLK];
    {
        #pragma clang fp contract(off)
        const float * qrow = a.q + ((size_t) h * a.rows + (rlive ? row : 0)) * HD + 8 * g;
        const uint32_t qmask = rlive ? 0xffffffffu : 0u;
        const float qs = a.qmode == 0 ? 1.0f : a.scale;
        #pragma unroll
        for (int s = 0; s < NBLK; s++) {
            const pa_f4 x0 = __builtin_bit_cast(pa_f4, __builtin_bit_cast(pa_u4, *(const pa_f4 *) (qrow + 32 * s)) & qmask);
            const pa_f4 x1 = __builtin_bit_cast(pa_f4, __builtin_bit_cast(pa_u4, *(const pa_f4 *) (qrow + 32 * s + 4)) & qmask);
            mm_h8 f;
            if constexpr (EX) {
                float am = fmaxf(fmaxf(fmaxf(fabsf(x0[0]), fabsf(x0[1])), fmaxf(fabsf(x0[2]), fabsf(x0[3]))),
                                 fmaxf(fmaxf(fabsf(x1[0]), fabsf(x1[1])), fmaxf(fabsf(x1[2]), fabsf(x1[3]))));
                am = mm_max32(m2_max16(am));
                const float d = am / 127.0f;
                const float id = d != 0.0f ? 1.0f / d : 0.0f;
                const float dq = (float) (_Float16) d * (a.scale * MM_LOG2E);
                const int sb = dq > 0.0f ? min(14, 3 - __builtin_amdgcn_frexp_expf(dq) + 1) : 0;
                const float v = __builtin_amdgcn_ldexpf(dq, sb);
                const _Float16 hi = (_Float16) v, lo = (_Float16) (v - (float) hi);
                dqw[s] = g == 0 ? (uint32_t) __builtin_bit_cast(uint16_t, hi) | ((uint32_t) __builtin_bit_cast(uint16_t, lo) << 16) : 0u;
                #pragma unroll
                for (int t = 0; t < 4; t++) {
                    f[t] = (_Float16) __builtin_amdgcn_ldexpf(roundf(x0[t] * id), -sb);
                    f[t + 4] = (_Float16) __builtin_amdgcn_ldexpf(roundf(x1[t] * id), -sb);
                }
            } else {
                dqw[s] = 0u;
                #pragma unroll
                for (int t = 0; t < 4; t++) {
                    f[t] = (_Float16) pa_f32(x0[t] * qs);            // f2h(q * scale)
                    f[t + 4] = (_Float16) pa_f32(x1[t] * qs);
                }
            }
            Qf[s] = f;
        }
    }

    store_tile(R[0], 0);
    load_tile(R[0], t0 + NB, ntiles > NB);
    mm_lds_barrier();

    pa_f4 O[HD / 16];
    #pragma unroll
    for (int db = 0; db < HD / 16; db++) O[db] = (pa_f4){};
    float mref = -INFINITY, mx = -INFINITY, lsum = 0.0f;
    const float sm = a.qmode == 0 && FMT == 0 ? a.scale * MM_LOG2E : MM_LOG2E;   // score -> base-2 logit (!EX)
    float mc = 0.0f;                                                 // EX: the scores' offset, mref once finite (0 before)
    const mm_h2 one2 = {(_Float16) 1.0f, (_Float16) 1.0f};

    auto compute = [&](int stage, int nvalid) {
        const char * Kt = smem + stage * M2_STAGE;
        const char * Vt = Kt + M2_KT;
        __builtin_amdgcn_s_waitcnt(0xc07f);                          // lgkmcnt(0): the stores and any scalar load done
        // ---- S^T = K Q'^T: the two key halves' chains interleaved, K read four steps ahead
        pa_f4 S[2] = {(pa_f4){}, (pa_f4){}};
        constexpr int KA = EX ? 1 : (NBLK < 4 ? NBLK : 4);           // K read KA steps ahead (EX holds more registers)
        mm_h8 kf[2][KA];
        auto k_read = [&](int s) {
            #pragma unroll
            for (int kh = 0; kh < 2; kh++) kf[kh][s % KA] = *(const mm_h8 *) (Kt + (16 * kh + n) * M2_KST + 2 * (32 * s + 8 * g));
        };
        #pragma unroll
        for (int s = 0; s < KA; s++) k_read(s);
        if constexpr (EX) {
            // per block s and key half kh: the integer dot times 2^-s_b, the scale product dk_s(key) * (hi + lo)(row)
            // (dk_s at k = 0 and 1 of A in lanes g = 0, the row's pair at k = 0 and 1 of B), their product summed in
            // block order from -mc: the base-2 logit minus the reference max
            const uint32_t gmask = g == 0 ? 0xffffffffu : 0u;
            uint32_t dk2[2];                                         // key 16 kh + n's fp16 scales of blocks s, s + 1
            #pragma unroll
            for (int s = 0; s < NBLK; s++) {
                if ((s & 1) == 0) {
                    #pragma unroll
                    for (int kh = 0; kh < 2; kh++)
                        dk2[kh] = *(const uint32_t *) (Kt + M2_KT + M2_VT + 2 * NBLK * (16 * kh + n) + 2 * s);
                }
                #pragma unroll
                for (int kh = 0; kh < 2; kh++) {
                    const pa_f4 Sb = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[kh][s % KA], Qf[s], (pa_f4){}, 0, 0, 0);
                    const uint32_t dkw = pa_perm(0u, dk2[kh], (s & 1) ? 0x03020302u : 0x01000100u) & gmask;
                    uint32_t dq = dqw[s];
                    asm volatile("" : "+v"(dq));                     // the operand tuple built here, not held across
                                                                     // tiles (8 tuples of 4 registers would spill)
                    const pa_f4 Pb = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mm_h8, (pa_u4){dkw, 0u, 0u, 0u}),
                                                                            __builtin_bit_cast(mm_h8, (pa_u4){dq, 0u, 0u, 0u}),
                                                                            (pa_f4){}, 0, 0, 0);
                    #pragma unroll
                    for (int i = 0; i < 4; i++) S[kh][i] = fmaf(Pb[i], Sb[i], s == 0 ? -mc : S[kh][i]);
                }
                if (s + KA < NBLK) k_read(s + KA);
                __builtin_amdgcn_sched_barrier(0);                   // one block at a time (registers)
            }
        } else {
            #pragma unroll
            for (int s = 0; s < NBLK; s++) {
                #pragma unroll
                for (int kh = 0; kh < 2; kh++) S[kh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[kh][s % KA], Qf[s], S[kh], 0, 0, 0);
                if (s + KA < NBLK) k_read(s + KA);
            }
        }
        if (nvalid < 32) {                                           // keys 16 kh + 4 g + i past the page's end
            #pragma unroll
            for (int kh = 0; kh < 2; kh++)
                #pragma unroll
                for (int i = 0; i < 4; i++)
                    if (16 * kh + 4 * g + i >= nvalid) S[kh][i] = -INFINITY;
        }
        float tm = fmaxf(fmaxf(fmaxf(S[0][0], S[0][1]), fmaxf(S[0][2], S[0][3])), fmaxf(fmaxf(S[1][0], S[1][1]), fmaxf(S[1][2], S[1][3])));
        tm = EX ? mm_max32(m2_max16(tm)) + mc : mm_max32(m2_max16(tm)) * sm;   // row n's tile max, base 2
        if (__builtin_amdgcn_ballot_w64(tm > mref + MM_PMAX)) {
            const float mn = fmaxf(mref, tm);
            const float alpha = mref == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mref - mn);
            #pragma unroll
            for (int db = 0; db < HD / 16; db++) O[db] *= alpha;
            lsum *= alpha;
            mref = mn;
            if constexpr (EX) {                                      // rebase this tile's scores to the new offset
                const float dl = mn - mc;
                #pragma unroll
                for (int kh = 0; kh < 2; kh++)
                    #pragma unroll
                    for (int i = 0; i < 4; i++) S[kh][i] -= dl;
                mc = mn;
            }
        }
        mx = fmaxf(mx, tm);
        mm_h8 P;
        #pragma unroll
        for (int kh = 0; kh < 2; kh++)
            #pragma unroll
            for (int i = 0; i < 4; i++)
                P[4 * kh + i] = (_Float16) __builtin_amdgcn_exp2f(EX ? S[kh][i] : fmaf(S[kh][i], sm, -mref));
        #pragma unroll
        for (int t = 0; t < 8; t += 2) {                             // the row sum of the fp16 P the PV MFMAs use
            const mm_h2 pp = {P[t], P[t + 1]};
            lsum = __builtin_amdgcn_fdot2(pp, one2, lsum, false);
        }
        // ---- O^T += V^T P^T per 16-dim block: lane (g, L) of a transposing read addresses key 16 r + 4 g + L / 4,
        // dims 16 db + 4 (L % 4) .. +3; lane (g, s) then holds dim 16 db + s of keys 16 r + 4 g + j (j < 4)
        const char * vrow = Vt + (4 * g + (n >> 2)) * M2_VST + 2 * 4 * (n & 3);
        #pragma unroll
        for (int db = 0; db < HD / 16; db++) {
            const pa_h4 x0 = __builtin_bit_cast(pa_h4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((MM_LDS mm_tr4 *) (vrow + 32 * db)));
            const pa_h4 x1 = __builtin_bit_cast(pa_h4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((MM_LDS mm_tr4 *) (vrow + 16 * M2_VST + 32 * db)));
            const mm_h8 va = __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
            O[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, P, O[db], 0, 0, 0);
        }
    };
    auto step = [&](uint32_t t, MmRaw<FMT> (&Rn)[UPT]) {
        const int stage = t & 1;
        const uint32_t tau = t0 + t, tn = tau + 1 + NB;              // this tile; the one loaded now
        cc.seek(a, tau);
        const int nvalid = (int) min(32u, cc.nk - 32 * (tau - cc.tb));
        const bool nlive = t + 1 + NB < ntiles;
        if (nlive) cl.seek(a, tn);
        store_tile(Rn, stage ^ 1);
        load_tile(Rn, tn, nlive);
        if (wlive) compute(stage, nvalid);
        mm_lds_barrier();
    };
    uint32_t t = 0;                                                  // tile t + 1 is in R[(t + 1) % NB]
    for (; t + NB <= ntiles; t += NB) {
        #pragma unroll
        for (int k = 0; k < NB; k++) step(t + k, R[(k + 1) % NB]);
    }
    #pragma unroll
    for (int k = 0; k < NB - 1; k++)
        if (t + k < ntiles) step(t + k, R[(k + 1) % NB]);

    // ---- row n's result: sum over its 4 lanes, O rebased from the reference max to the exact one
    const float lt = mm_sum32(m2_sum16(lsum));
    const float f = mref == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mref - mx);
    if (!rlive) return;
    const bool direct = a.n_chunks == 1 && a.fused;
    float * dst = direct ? a.O + ((size_t) h * a.rows + row) * HD
                         : a.po + (((size_t) h * a.qr + row) * a.slots + a.slot0 + c) * HD;
    #pragma unroll
    for (int db = 0; db < HD / 16; db++) *(pa_f4 *) (dst + 16 * db + 4 * g) = O[db] * f;
    if (g == 0) {
        if (direct) {
            a.m[(size_t) h * a.rows + row] = mx == -INFINITY ? -INFINITY : mx * PA_LN2;
            a.l[(size_t) h * a.rows + row] = lt * f;
        } else {
            a.pml[((size_t) h * a.qr + row) * a.slots + a.slot0 + c] = make_float2(mx, lt * f);
        }
    }
}

template <int HD, int WPS>
static hipError_t launch_m16(int fmt, bool skip, bool ex, const AttnArgs & a, uint32_t grid, hipStream_t st, hipEvent_t ev0,
                             hipEvent_t ev1) {
    switch (fmt * 4 + (skip ? 2 : 0) + (ex ? 1 : 0)) {
        case 0: hipExtLaunchKernelGGL((mma256_kernel<HD, 0, false, false, WPS>), dim3(grid), dim3(256), 0, st, ev0, ev1, 0, a); break;
        case 2: hipExtLaunchKernelGGL((mma256_kernel<HD, 0, true, false, WPS>), dim3(grid), dim3(256), 0, st, ev0, ev1, 0, a); break;
        case 4: hipExtLaunchKernelGGL((mma256_kernel<HD, 1, false, false, WPS>), dim3(grid), dim3(256), 0, st, ev0, ev1, 0, a); break;
        case 5: hipExtLaunchKernelGGL((mma256_kernel<HD, 1, false, true, WPS>), dim3(grid), dim3(256), 0, st, ev0, ev1, 0, a); break;
        case 6: hipExtLaunchKernelGGL((mma256_kernel<HD, 1, true, false, WPS>), dim3(grid), dim3(256), 0, st, ev0, ev1, 0, a); break;
        case 7: hipExtLaunchKernelGGL((mma256_kernel<HD, 1, true, true, WPS>), dim3(grid), dim3(256), 0, st, ev0, ev1, 0, a); break;
        case 8: hipExtLaunchKernelGGL((mma256_kernel<HD, 2, false, false, WPS>), dim3(grid), dim3(256), 0, st, ev0, ev1, 0, a); break;
        case 9: hipExtLaunchKernelGGL((mma256_kernel<HD, 2, false, true, WPS>), dim3(grid), dim3(256), 0, st, ev0, ev1, 0, a); break;
        case 10: hipExtLaunchKernelGGL((mma256_kernel<HD, 2, true, false, WPS>), dim3(grid), dim3(256), 0, st, ev0, ev1, 0, a); break;
        case 11: hipExtLaunchKernelGGL((mma256_kernel<HD, 2, true, true, WPS>), dim3(grid), dim3(256), 0, st, ev0, ev1, 0, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ggml's query rounding over quantized K takes the exact block dots; f16 queries (and f16 K) the fp16 operands
hipError_t launch_mma256(int fmt, bool skip, const AttnArgs & a, uint32_t grid, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    return launch_m16<256, 2>(fmt, skip, a.qmode == 0 && fmt != 0, a, grid, st, ev0, ev1);
}

}  // namespace pa_hip
