// pa_attn.hip - split-K partial attention over quantized K/V pages, fp16 MFMA (gfx950).
//
// One workgroup = one KV head x one block of 16*RT*WR query rows x one chunk of keys of one page. Per tile of NB keys the
// workgroup dequantizes K into LDS row-major (fp16, [key][dim]) and V transposed ([dim][key]) - the int8/int4 -> fp16
// conversion runs once per tile and feeds every row of the block. Each wave then computes, per 32-key step,
//   S^T (keys x rows) = K . Q^T with v_mfma_f32_16x16x32_f16 (A = K rows from LDS, B = Q^T held in registers),
// which leaves lane (g, n) with row n's scores of keys 4g..4g+3 (+16): exactly the B operand of
//   O^T (dims x rows) += V^T . P^T,
// so the probabilities never leave registers, and the running max / sum of row n live in the lanes that own row n.
// Online softmax runs in base 2 (the softmax scale and log2 e are folded into one multiply). WK waves may split the
// keys of a tile; their states are merged through LDS at the end. Each workgroup writes one split-K slot
// (O^T unnormalised, m in base-2 units, l); pa_merge_kernel folds the slots.
//
// Reference roles: pa_attn_big + pa_big_load (pa-metal.mm:379-487: per (row tile, KV head, key chunk), dequant a K/V
// block, S = QK^T, online softmax with key masking, O = alpha O + PV, write a slot) and pa_merge / pa_merge_big
// (pa-metal.mm:137-159, 490-524: M = max, skip -inf slots, w = exp(m_c - M), O = sum w O_c, L = sum w l_c).
#include "pa_attn.h"
#include "pa_common.h"

namespace pa_hip {

// ---------------------------------------------------------------- tile loaders (HBM -> registers -> LDS fp16)
template <int HD, int FMT, int NB, int NT>
__device__ __forceinline__ void load_k_tile(_Float16 * __restrict__ Ks, float * __restrict__ Ksc, const uint8_t * __restrict__ kb,
                                            uint32_t rs, uint32_t jt, int nvalid, int tid, float s_mul) {
    // K stays exact: the quants (q8_0: q, q4_0: nib - 8) as integer-valued fp16, and d * s_mul per (block, key) in
    // Ksc[blk][key], applied to each block's fp32 partial dot after the MFMA (the order ggml's q8_0 x q8_0 dot uses).
    constexpr int NBLK = HD / 32, KS = HD + 8;
    #pragma unroll
    for (int it0 = 0; it0 < NB * NBLK; it0 += NT) {
        const int it = it0 + tid;
        if (NB * NBLK % NT != 0 && it >= NB * NBLK) break;
        const int key = it / NBLK, blk = it % NBLK;
        pa_u4 o[4] = {};
        float sc = 0.0f;
        if (key < nvalid) {
            const uint8_t * src = kb + (size_t) (jt + key) * rs;
            if constexpr (FMT == 1) {
                src += blk * 34;
                sc = pa_f16_bits_to_f32(pa_ld<uint16_t>(src)) * s_mul;
                const pa_u4 q0 = pa_ld<pa_u4>(src + 2), q1 = pa_ld<pa_u4>(src + 18);
                const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
                #pragma unroll
                for (int w = 0; w < 8; w++) {
                    uint32_t lo, hi;
                    pa_int_q8x4(qw[w], lo, hi);
                    o[w / 2][(w % 2) * 2 + 0] = lo;
                    o[w / 2][(w % 2) * 2 + 1] = hi;
                }
            } else if constexpr (FMT == 2) {
                src += blk * 18;
                sc = pa_f16_bits_to_f32(pa_ld<uint16_t>(src)) * s_mul;
                const pa_u4 q = pa_ld<pa_u4>(src + 2);
                const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
                #pragma unroll
                for (int w = 0; w < 4; w++) {   // bytes 4w..4w+3: low nibbles = elements 4w.., high = 16+4w..
                    uint32_t lo, hi;
                    pa_int_nib4(qw[w] & 0x0f0f0f0fu, lo, hi);
                    o[w / 2][(w % 2) * 2 + 0] = lo;
                    o[w / 2][(w % 2) * 2 + 1] = hi;
                    pa_int_nib4((qw[w] >> 4) & 0x0f0f0f0fu, lo, hi);
                    o[2 + w / 2][(w % 2) * 2 + 0] = lo;
                    o[2 + w / 2][(w % 2) * 2 + 1] = hi;
                }
            } else {
                src += blk * 64;
                sc = s_mul;
                #pragma unroll
                for (int c = 0; c < 4; c++) o[c] = pa_ld<pa_u4>(src + 16 * c);
            }
        }
        pa_u4 * dst = (pa_u4 *) (Ks + key * KS + blk * 32);
        #pragma unroll
        for (int c = 0; c < 4; c++) dst[c] = o[c];
        Ksc[blk * NB + key] = sc;
    }
}

// V tile, transposed: Vt[dim][key] (row stride NB+4 halves). A work item is (key pair, 32-dim block): the two keys'
// values of one dim are packed into one dword, so the LDS writes are 4-byte and the PV operand reads 8-byte runs of keys.
template <int HD, int FMT, int NB, int NT>
__device__ __forceinline__ void load_v_tile(_Float16 * __restrict__ Vt, const uint8_t * __restrict__ vb, uint32_t rs,
                                            uint32_t jt, int nvalid, int tid) {
    constexpr int NBLK = HD / 32, VS = NB + 4;
    constexpr int NIT = NB / 2 * NBLK;
    #pragma unroll
    for (int it0 = 0; it0 < NIT; it0 += NT) {
        const int it = it0 + tid;
        if (NIT % NT != 0 && it >= NIT) break;
        const int kp = it / NBLK, blk = it % NBLK, k0 = 2 * kp;
        uint32_t * col = (uint32_t *) (Vt + (blk * 32) * VS + k0);   // dim blk*32 + d at col + d*VS/2
        const bool v0 = k0 < nvalid, v1 = k0 + 1 < nvalid;
        const uint8_t * s0 = vb + (size_t) (jt + k0) * rs, * s1 = s0 + rs;
        if constexpr (FMT == 1) {
            pa_u4 a0 = {}, a1 = {}, b0 = {}, b1 = {};
            uint16_t da = 0, dbb = 0;
            if (v0) { s0 += blk * 34; da = pa_ld<uint16_t>(s0); a0 = pa_ld<pa_u4>(s0 + 2); a1 = pa_ld<pa_u4>(s0 + 18); }
            if (v1) { s1 += blk * 34; dbb = pa_ld<uint16_t>(s1); b0 = pa_ld<pa_u4>(s1 + 2); b1 = pa_ld<pa_u4>(s1 + 18); }
            const pa_h2 d2 = {__builtin_bit_cast(_Float16, da), __builtin_bit_cast(_Float16, dbb)};
            const pa_h2 bias = {(_Float16) 1152.0f, (_Float16) 1152.0f};
            const uint32_t xa[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            const uint32_t xb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
            #pragma unroll
            for (int w = 0; w < 8; w++) {
                const uint32_t x0 = xa[w] ^ 0x80808080u, x1 = xb[w] ^ 0x80808080u;
                #pragma unroll
                for (int e = 0; e < 4; e++)
                    col[(4 * w + e) * (VS / 2)] = pa_as_u32((pa_as_h2(pa_pair_byte(x1, x0, e)) - bias) * d2);
            }
        } else if constexpr (FMT == 2) {
            pa_u4 a = {}, b = {};
            uint16_t da = 0, dbb = 0;
            if (v0) { s0 += blk * 18; da = pa_ld<uint16_t>(s0); a = pa_ld<pa_u4>(s0 + 2); }
            if (v1) { s1 += blk * 18; dbb = pa_ld<uint16_t>(s1); b = pa_ld<pa_u4>(s1 + 2); }
            const pa_h2 d2 = {__builtin_bit_cast(_Float16, da), __builtin_bit_cast(_Float16, dbb)};
            const pa_h2 bias = {(_Float16) 1032.0f, (_Float16) 1032.0f};
            const uint32_t xa[4] = {a.x, a.y, a.z, a.w}, xb[4] = {b.x, b.y, b.z, b.w};
            #pragma unroll
            for (int w = 0; w < 4; w++) {
                const uint32_t l0 = xa[w] & 0x0f0f0f0fu, l1 = xb[w] & 0x0f0f0f0fu;
                const uint32_t h0 = (xa[w] >> 4) & 0x0f0f0f0fu, h1 = (xb[w] >> 4) & 0x0f0f0f0fu;
                #pragma unroll
                for (int e = 0; e < 4; e++) {
                    col[(4 * w + e) * (VS / 2)] = pa_as_u32((pa_as_h2(pa_pair_byte(l1, l0, e)) - bias) * d2);
                    col[(16 + 4 * w + e) * (VS / 2)] = pa_as_u32((pa_as_h2(pa_pair_byte(h1, h0, e)) - bias) * d2);
                }
            }
        } else {
            pa_u4 a[4] = {}, b[4] = {};
            if (v0) { s0 += blk * 64; for (int c = 0; c < 4; c++) a[c] = pa_ld<pa_u4>(s0 + 16 * c); }
            if (v1) { s1 += blk * 64; for (int c = 0; c < 4; c++) b[c] = pa_ld<pa_u4>(s1 + 16 * c); }
            #pragma unroll
            for (int w = 0; w < 16; w++) {   // dword w = dims 2w, 2w+1
                const uint32_t x0 = a[w / 4][w % 4], x1 = b[w / 4][w % 4];
                col[(2 * w) * (VS / 2)] = pa_perm(x1, x0, 0x05040100u);
                col[(2 * w + 1) * (VS / 2)] = pa_perm(x1, x0, 0x07060302u);
            }
        }
    }
}

// ---------------------------------------------------------------- the attention kernel
template <int HD, int FMT, int RT, int WR, int WK, int NB>
__global__ __launch_bounds__(64 * WR * WK) void attn_kernel(const AttnArgs a) {
    constexpr int NT = 64 * WR * WK;
    constexpr int KS = HD + 8, VS = NB + 4;
    constexpr int ND = HD / 16;        // 16-dim blocks of O^T
    constexpr int NKD = HD / 32;       // 32-dim k-steps of QK
    constexpr int KPW = NB / WK;       // keys of a tile per wave
    static_assert(KPW % 32 == 0, "each wave needs whole 32-key steps");
    constexpr int ROWS_WG = 16 * RT * WR;
    constexpr int TILE_LDS = (NB * KS + HD * VS) * 2 + NKD * NB * 4;
    constexpr int COMB_LDS = WK > 1 ? WK * ROWS_WG * (HD + 2) * 4 : 0;
    constexpr int LDS = TILE_LDS > COMB_LDS ? TILE_LDS : COMB_LDS;
    __shared__ __attribute__((aligned(16))) char smem[LDS];
    _Float16 * Ks = (_Float16 *) smem;
    _Float16 * Vt = Ks + NB * KS;
    float * Ksc = (float *) (Vt + HD * VS);   // [NKD][NB]: K block scale * s_mul

    // ---- which (chunk, head, row block). Items are numbered chunk-major (row block fastest) and XCD x (= blockIdx % 8 in
    // the dispatch order) takes the contiguous item range [x*T8, (x+1)*T8): the heads of one chunk (which share cache
    // lines of the same key rows) and the row blocks of one head (which read the same K/V) stay in one XCD's L2.
    const uint32_t b = blockIdx.x, xcd = b % 8, local = b / 8;
    const uint32_t t8 = (a.n_items + 7) / 8;
    const uint32_t w = xcd * t8 + local;
    if (local >= t8 || w >= a.n_items) return;
    const uint32_t rb = w % a.nrb, h = (w / a.nrb) % a.nkv, c = w / (a.nrb * a.nkv);
    const uint32_t key_lo = c * a.chunk, key_hi = min(a.pstart[a.n_pages], key_lo + a.chunk);
    uint32_t p = 0;
    while (p + 1 < a.n_pages && a.pstart[p + 1] <= key_lo) p++;

    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int wr = wave % WR, wk = wave / WR, g = lane / 16, n = lane % 16;
    const uint32_t row_base = rb * ROWS_WG + wr * RT * 16;   // first row of this wave's row tiles (within the head)

    // ---- Q^T fragments (B operand of QK): lane (g, n) holds row n, dims 32kd + 8g .. +7, as hi + lo fp16 pairs whose sum
    // is the prepared query exactly (q8_0-rounded in ggml mode); lo is all zero when a.hilo == 0
    pa_h8 qh[RT][NKD], ql[RT][NKD];
    #pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const size_t off = ((size_t) h * a.qr + row_base + rt * 16 + n) * HD + 8 * g;
        #pragma unroll
        for (int kd = 0; kd < NKD; kd++) {
            qh[rt][kd] = *(const pa_h8 *) (a.q16 + off + 32 * kd);
            ql[rt][kd] = *(const pa_h8 *) (a.q16 + a.q16_lo + off + 32 * kd);
        }
    }
    const bool hilo = a.hilo != 0;
    pa_f4 o[RT][ND];
    float mrow[RT], lrow[RT];
    #pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        mrow[rt] = -INFINITY; lrow[rt] = 0.0f;
        #pragma unroll
        for (int d = 0; d < ND; d++) o[rt][d] = (pa_f4){0.f, 0.f, 0.f, 0.f};
    }
    const float s_mul = a.s_mul;

    for (; p < a.n_pages && a.pstart[p] < key_hi; p++) {
      const uint32_t j0 = max(key_lo, a.pstart[p]) - a.pstart[p], j1 = min(key_hi, a.pstart[p + 1]) - a.pstart[p];
      const uint8_t * kb = a.kp[p] + (size_t) h * a.hb;
      const uint8_t * vb = a.vp[p] + (size_t) h * a.hb;
      for (uint32_t jt = j0; jt < j1; jt += NB) {
        const int nvalid = (int) min((uint32_t) NB, j1 - jt);
        __syncthreads();
        load_k_tile<HD, FMT, NB, NT>(Ks, Ksc, kb, a.rs, jt, nvalid, tid, s_mul);
        load_v_tile<HD, FMT, NB, NT>(Vt, vb, a.rs, jt, nvalid, tid);
        __syncthreads();
        #pragma unroll
        for (int ks = 0; ks < KPW / 32; ks++) {
            const int kbase = wk * KPW + ks * 32;                 // first key of this 32-key step within the tile
            if (kbase >= nvalid) break;
            // S^T = K . Q^T for two 16-key subtiles, one MFMA (two with the lo half) per 32-dim block: exact integer-scaled
            // partial dots, combined in fp32 with the block's K scale (already times s_mul: base-2 logits come out)
            pa_f4 s[RT][2];
            #pragma unroll
            for (int rt = 0; rt < RT; rt++) s[rt][0] = s[rt][1] = (pa_f4){0.f, 0.f, 0.f, 0.f};
            #pragma unroll
            for (int kd = 0; kd < NKD; kd++) {
                const pa_h8 k0 = *(const pa_h8 *) (Ks + (kbase + n) * KS + 32 * kd + 8 * g);
                const pa_h8 k1 = *(const pa_h8 *) (Ks + (kbase + 16 + n) * KS + 32 * kd + 8 * g);
                const pa_f4 d0 = *(const pa_f4 *) (Ksc + kd * NB + kbase + 4 * g);
                const pa_f4 d1 = *(const pa_f4 *) (Ksc + kd * NB + kbase + 16 + 4 * g);
                #pragma unroll
                for (int rt = 0; rt < RT; rt++) {
                    const pa_f4 z = {0.f, 0.f, 0.f, 0.f};
                    pa_f4 a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, qh[rt][kd], z, 0, 0, 0);
                    pa_f4 a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, qh[rt][kd], z, 0, 0, 0);
                    if (hilo) {
                        a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, ql[rt][kd], a0, 0, 0, 0);
                        a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, ql[rt][kd], a1, 0, 0, 0);
                    }
                    s[rt][0] += d0 * a0;
                    s[rt][1] += d1 * a1;
                }
            }
            // V^T operand: lane (g, n) = dim 16*db + n, keys kbase + 4g..+3 and kbase + 16 + 4g..+3
            pa_h8 pf[RT];
            #pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                float v[8];
                #pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int k0i = kbase + 4 * g + i, k1i = kbase + 16 + 4 * g + i;
                    v[i] = k0i < nvalid ? s[rt][0][i] : -INFINITY;
                    v[4 + i] = k1i < nvalid ? s[rt][1][i] : -INFINITY;
                }
                float tm = v[0];
                #pragma unroll
                for (int i = 1; i < 8; i++) tm = fmaxf(tm, v[i]);
                tm = pa_wave_max16x4(tm);
                const float mn = fmaxf(mrow[rt], tm);
                const float ms = mn == -INFINITY ? 0.0f : mn;
                const float alpha = __builtin_amdgcn_exp2f(mrow[rt] - ms);
                float sum = 0.0f;
                #pragma unroll
                for (int i = 0; i < 8; i++) { v[i] = __builtin_amdgcn_exp2f(v[i] - ms); sum += v[i]; }
                lrow[rt] = lrow[rt] * alpha + sum;
                mrow[rt] = mn;
                #pragma unroll
                for (int d = 0; d < ND; d++) o[rt][d] *= alpha;
                #pragma unroll
                for (int i = 0; i < 8; i++) pf[rt][i] = (_Float16) v[i];
            }
            #pragma unroll
            for (int db = 0; db < ND; db++) {
                const _Float16 * vr = Vt + (16 * db + n) * VS + kbase + 4 * g;
                const pa_h4 va = *(const pa_h4 *) vr, vbv = *(const pa_h4 *) (vr + 16);
                const pa_h8 vv = {va[0], va[1], va[2], va[3], vbv[0], vbv[1], vbv[2], vbv[3]};
                #pragma unroll
                for (int rt = 0; rt < RT; rt++) o[rt][db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vv, pf[rt], o[rt][db], 0, 0, 0);
            }
        }
      }
    }

    // ---- per-row sums over the 4 lane groups
    #pragma unroll
    for (int rt = 0; rt < RT; rt++) lrow[rt] = pa_wave_sum16x4(lrow[rt]);

    const uint32_t slot = a.slot0 + c;
    float * po = a.po + ((size_t) slot * a.nkv + h) * a.qr * HD;
    float2 * pml = a.pml + ((size_t) slot * a.nkv + h) * a.qr;
    if constexpr (WK == 1) {
        #pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const uint32_t row = row_base + rt * 16 + n;
            if (row >= a.rows) continue;
            #pragma unroll
            for (int db = 0; db < ND; db++) *(pa_f4 *) (po + (size_t) row * HD + 16 * db + 4 * g) = o[rt][db];
            if (g == 0) pml[row] = make_float2(mrow[rt], lrow[rt]);
        }
    } else {
        // merge the WK key-split states of the same rows through LDS
        __syncthreads();
        float * cO = (float *) smem;                                    // [WK][ROWS_WG][HD]
        float2 * cML = (float2 *) (cO + WK * ROWS_WG * HD);            // [WK][ROWS_WG]
        #pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const int lr = (wr * RT + rt) * 16 + n;
            #pragma unroll
            for (int db = 0; db < ND; db++) *(pa_f4 *) (cO + ((size_t) wk * ROWS_WG + lr) * HD + 16 * db + 4 * g) = o[rt][db];
            if (g == 0) cML[wk * ROWS_WG + lr] = make_float2(mrow[rt], lrow[rt]);
        }
        __syncthreads();
        for (int e = tid; e < ROWS_WG * (HD / 4); e += NT) {
            const int lr = e / (HD / 4), d4 = e % (HD / 4);
            const uint32_t row = rb * ROWS_WG + lr;
            if (row >= a.rows) continue;
            float M = -INFINITY;
            #pragma unroll
            for (int w = 0; w < WK; w++) M = fmaxf(M, cML[w * ROWS_WG + lr].x);
            const float Ms = M == -INFINITY ? 0.0f : M;
            pa_f4 acc = {0.f, 0.f, 0.f, 0.f};
            float L = 0.0f;
            #pragma unroll
            for (int w = 0; w < WK; w++) {
                const float2 ml = cML[w * ROWS_WG + lr];
                const float wt = __builtin_amdgcn_exp2f(ml.x - Ms);
                L += wt * ml.y;
                acc += wt * *(const pa_f4 *) (cO + ((size_t) w * ROWS_WG + lr) * HD + 4 * d4);
            }
            *(pa_f4 *) (po + (size_t) row * HD + 4 * d4) = acc;
            if (d4 == 0) pml[row] = make_float2(M, L);
        }
    }
}

// ---------------------------------------------------------------- split-K fold
// One workgroup per output row; thread t folds dims 4*(t % (HD/4)) over slots t / (HD/4), t / (HD/4) + SG, ...
template <int HD>
__global__ __launch_bounds__(256) void merge_kernel(const MergeArgs a) {
    constexpr int TPR = HD / 4, SG = 256 / TPR;
    __shared__ pa_f4 red[SG][TPR];
    __shared__ float redl[SG];
    const uint32_t r = blockIdx.x;                   // output row = h*rows + i
    const uint32_t h = r / a.rows, i = r % a.rows;
    const int t = threadIdx.x, d4 = t % TPR, sg = t / TPR;
    const size_t stride = (size_t) a.nkv * a.qr;     // rows between slots
    const size_t pr = (size_t) h * a.qr + i;
    float M = -INFINITY;
    for (uint32_t s = 0; s < a.n_slots; s++) M = fmaxf(M, a.pml[s * stride + pr].x);
    const float Ms = M == -INFINITY ? 0.0f : M;
    pa_f4 acc = {0.f, 0.f, 0.f, 0.f};
    float L = 0.0f;
    for (uint32_t s = sg; s < a.n_slots; s += SG) {
        const float2 ml = a.pml[s * stride + pr];
        const float w = __builtin_amdgcn_exp2f(ml.x - Ms);   // ml.x = -inf -> 0 (an empty slot)
        L += w * ml.y;
        acc += w * *(const pa_f4 *) (a.po + (s * stride + pr) * HD + 4 * d4);
    }
    red[sg][d4] = acc;
    if (d4 == 0) redl[sg] = L;
    __syncthreads();
    if (sg == 0) {
        for (int q = 1; q < SG; q++) { acc += red[q][d4]; if (d4 == 0) L += redl[q]; }
        *(pa_f4 *) (a.O + (size_t) r * HD + 4 * d4) = acc;
        if (d4 == 0) { a.m[r] = M == -INFINITY ? -INFINITY : M * PA_LN2; a.l[r] = L; }
    }
}

// ---------------------------------------------------------------- Q preparation
// One thread per (row, 32-block): Q fp32 [nkv][rows][HD] -> hi [nkv][qr][HD] and lo (at +q16_lo) fp16 with hi + lo equal to
// the query value the dot product must see (rows >= `rows` zero).
// PA_QMODE_GGML, quantized K: q8_0 of the block (d = amax/127, id = 1/d, q = roundf(x*id), d -> fp16:
// quantize_row_q8_0_ref), value t = d16 * q (exact in fp32), hi = f16(t), lo = f16(t - hi) - exact, so the fp16 MFMA
// against integer K reproduces ggml's integer block dot. PA_QMODE_GGML, f16 K: f16(x) (ggml's vec_dot_type for f16 K).
// PA_QMODE_F16: f16(x*scale) (the reference engines). lo = 0 in the last two.
__global__ __launch_bounds__(256) void qprep_kernel(const QprepArgs a) {
    const uint32_t nblk = a.hd / 32;
    const uint32_t idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= a.nkv * a.qr * nblk) return;
    const uint32_t blk = idx % nblk, row = (idx / nblk) % a.qr, h = idx / nblk / a.qr;
    const size_t off = ((size_t) h * a.qr + row) * a.hd + blk * 32;
    _Float16 * hi = a.q16 + off, * lo = a.q16 + a.q16_lo + off;
    if (row >= a.rows) { for (int j = 0; j < 32; j++) hi[j] = lo[j] = (_Float16) 0.0f; return; }
    const float * x = a.q + ((size_t) h * a.rows + row) * a.hd + blk * 32;
    if (a.qmode == 0 && a.fmt != 0) {
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const float d16 = (float) (_Float16) d;
        for (int j = 0; j < 32; j++) {
            const float t = d16 * roundf(x[j] * id);
            const _Float16 th = (_Float16) t;
            hi[j] = th;
            lo[j] = (_Float16) (t - (float) th);
        }
    } else {
        const float mul = a.qmode == 0 ? 1.0f : a.scale;
        for (int j = 0; j < 32; j++) { hi[j] = (_Float16) (x[j] * mul); lo[j] = (_Float16) 0.0f; }
    }
}

// ggml quantize_row_q8_0_ref / quantize_row_q4_0_ref on the device, one thread per 32-block.
__global__ __launch_bounds__(256) void quantize_kernel(const float * __restrict__ x, uint8_t * __restrict__ y, int64_t nblk, int fmt) {
    const int64_t b = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (b >= nblk) return;
    const float * xb = x + b * 32;
    if (fmt == 1) {
        uint8_t * o = y + b * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(xb[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = __builtin_bit_cast(uint16_t, (_Float16) d);
        o[0] = (uint8_t) (dh & 0xff); o[1] = (uint8_t) (dh >> 8);
        for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t) (int8_t) roundf(xb[j] * id);
    } else {
        uint8_t * o = y + b * 18;
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < 32; j++) { const float v = xb[j]; if (amax < fabsf(v)) { amax = fabsf(v); mx = v; } }
        const float d = mx / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = __builtin_bit_cast(uint16_t, (_Float16) d);
        o[0] = (uint8_t) (dh & 0xff); o[1] = (uint8_t) (dh >> 8);
        for (int j = 0; j < 16; j++) {
            int q0 = (int8_t) (xb[j] * id + 8.5f), q1 = (int8_t) (xb[16 + j] * id + 8.5f);
            q0 = q0 > 15 ? 15 : q0;
            q1 = q1 > 15 ? 15 : q1;
            o[2 + j] = (uint8_t) (q0 | (q1 << 4));
        }
    }
}

// ---------------------------------------------------------------- launch table
template <int HD, int FMT, int RT, int WR, int WK, int NB>
static hipError_t launch_attn(const AttnArgs & a, uint32_t grid, hipStream_t st) {
    hipLaunchKernelGGL((attn_kernel<HD, FMT, RT, WR, WK, NB>), dim3(grid), dim3(64 * WR * WK), 0, st, a);
    return hipGetLastError();
}

template <int HD, int FMT>
static hipError_t launch_attn_cfg(int cfg, const AttnArgs & a, uint32_t grid, hipStream_t st) {
    if constexpr (HD == 256) {   // head dim 256 (the reference shape): at most 64 rows per workgroup (registers)
        if (cfg == CFG_DECODE) return launch_attn<HD, FMT, 1, 1, 2, 64>(a, grid, st);
        return launch_attn<HD, FMT, 1, 4, 1, 64>(a, grid, st);
    } else {
        switch (cfg) {
            case CFG_DECODE: return launch_attn<HD, FMT, 1, 1, 2, 64>(a, grid, st);
            case CFG_MID:    return launch_attn<HD, FMT, 1, 4, 1, 64>(a, grid, st);
            default:         return launch_attn<HD, FMT, 2, 4, 1, 64>(a, grid, st);   // verify / prefill
        }
    }
}

hipError_t launch_attention(int hd, int fmt, int cfg, const AttnArgs & a, uint32_t grid, hipStream_t st) {
    if (hd == 128) {
        if (fmt == 0) return launch_attn_cfg<128, 0>(cfg, a, grid, st);
        if (fmt == 1) return launch_attn_cfg<128, 1>(cfg, a, grid, st);
        if (fmt == 2) return launch_attn_cfg<128, 2>(cfg, a, grid, st);
    } else if (hd == 256) {
        if (fmt == 0) return launch_attn_cfg<256, 0>(cfg, a, grid, st);
        if (fmt == 1) return launch_attn_cfg<256, 1>(cfg, a, grid, st);
        if (fmt == 2) return launch_attn_cfg<256, 2>(cfg, a, grid, st);
    }
    return hipErrorInvalidValue;
}

void cfg_geometry(int cfg, int hd, int & rows_per_wg, int & nb) {
    nb = 64;
    if (cfg == CFG_DECODE) rows_per_wg = 16;
    else if (cfg == CFG_MID || hd == 256) rows_per_wg = 64;
    else rows_per_wg = 128;
}

hipError_t launch_merge(int hd, const MergeArgs & a, hipStream_t st) {
    const uint32_t grid = a.nkv * a.rows;
    if (hd == 128) hipLaunchKernelGGL(merge_kernel<128>, dim3(grid), dim3(256), 0, st, a);
    else if (hd == 256) hipLaunchKernelGGL(merge_kernel<256>, dim3(grid), dim3(256), 0, st, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_qprep(const QprepArgs & a, hipStream_t st) {
    const uint32_t n = a.nkv * a.qr * (a.hd / 32);
    hipLaunchKernelGGL(qprep_kernel, dim3((n + 255) / 256), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_quantize(int fmt, const float * x, void * y, int64_t n, hipStream_t st) {
    const int64_t nblk = n / 32;
    if (nblk == 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_kernel, dim3((uint32_t) ((nblk + 255) / 256)), dim3(256), 0, st, x, (uint8_t *) y, nblk, fmt);
    return hipGetLastError();
}

}  // namespace pa_hip
