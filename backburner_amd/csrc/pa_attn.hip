// pa_attn.hip - split-K partial attention over quantized K/V pages, fp16 MFMA (gfx950).
//
// One workgroup = one KV head x one block of 16*RT*WR query rows x one chunk of keys (a chunk may span pages). Per tile
// of NB keys (inside one page) the workgroup stages K into LDS row-major as exact integer-valued fp16 (the q8_0/q4_0
// quants) with the block scales in a small side array, and V transposed ([dim][key], fp16 d*q). The next tile's raw
// bytes are already in flight into registers while the current tile is computed. Each wave then computes, per 32-key
// step,
//   S^T (keys x rows) = K . Q^T with v_mfma_f32_16x16x32_f16, one MFMA per 32-dim block (= one quant block), and the
//   block's partial dot times d_k * scale * log2 e added in fp32 - the query is q8_0-rounded in-kernel (ggml's Q
//   handling) and held as an exact fp16 hi + lo pair, so the QK dot equals ggml's integer block dot;
//   O^T (dims x rows) += V^T . P^T,
// so lane (g, n) holds row n's scores of keys 4g..4g+3 (+16) - exactly the B operand of the PV MFMA - and the running
// max / sum of row n live in the lanes that own row n. Online softmax is in base 2. WK waves may split the keys of a
// tile; their states merge through LDS. Each workgroup then writes one split-K slot (O^T unnormalised, base-2 max, sum),
// which a merge kernel folds into the final (O, m, l); with one chunk the workgroup writes the final result directly.
// This kernel serves head dim 256 (the reference's compile-time shape); head dim 128 runs on dec_kernel / mma_kernel.
//
// Reference roles: pa_attn_big + pa_big_load (pa-metal.mm:379-487: per (row tile, KV head, key chunk), dequant a K/V
// block, S = QK^T, online softmax with key masking, O = alpha O + PV, write a slot) and pa_merge / pa_merge_big
// (pa-metal.mm:137-159, 490-524: M = max, skip -inf slots, w = exp(m_c - M), O = sum w O_c, L = sum w l_c).
#include "pa_attn.h"
#include "pa_common.h"

namespace pa_hip {

// ---------------------------------------------------------------- raw tile registers
// Words per 32-dim block item: q8_0 = fp16 scale + 32 bytes (9 dwords), q4_0 = scale + 16 bytes (5), f16 = 64 bytes (16).
template <int FMT> struct ItemWords { static constexpr int W = FMT == 1 ? 9 : FMT == 2 ? 5 : 16; };

template <int HD, int FMT, int NB, int NT> struct TileRegs {
    static constexpr int NBLK = HD / 32, W = ItemWords<FMT>::W;
    static constexpr int KIT = (NB * NBLK + NT - 1) / NT;        // K items (key, block) per thread
    static constexpr int VIT = (NB / 2 * NBLK + NT - 1) / NT;    // V items (key pair, block) per thread
    uint32_t k[KIT][W];
    uint32_t v[VIT][2][W];
};

template <int FMT>
__device__ __forceinline__ void load_item(uint32_t * w, const uint8_t * row, int blk) {
    if constexpr (FMT == 1) {
        const uint8_t * s = row + blk * 34;
        w[0] = pa_ld<uint16_t>(s);
        const pa_u4 a = pa_ld<pa_u4>(s + 2), b = pa_ld<pa_u4>(s + 18);
        w[1] = a.x; w[2] = a.y; w[3] = a.z; w[4] = a.w; w[5] = b.x; w[6] = b.y; w[7] = b.z; w[8] = b.w;
    } else if constexpr (FMT == 2) {
        const uint8_t * s = row + blk * 18;
        w[0] = pa_ld<uint16_t>(s);
        const pa_u4 a = pa_ld<pa_u4>(s + 2);
        w[1] = a.x; w[2] = a.y; w[3] = a.z; w[4] = a.w;
    } else {
        const uint8_t * s = row + blk * 64;
        #pragma unroll
        for (int c = 0; c < 4; c++) { const pa_u4 a = pa_ld<pa_u4>(s + 16 * c); w[4 * c] = a.x; w[4 * c + 1] = a.y; w[4 * c + 2] = a.z; w[4 * c + 3] = a.w; }
    }
}

// HBM -> registers for the tile of keys [jt, jt + nvalid) of one page (keys past nvalid read nothing, hold zeros)
template <int HD, int FMT, int NB, int NT>
__device__ __forceinline__ void load_tile(TileRegs<HD, FMT, NB, NT> & R, const uint8_t * __restrict__ kb, const uint8_t * __restrict__ vb,
                                          uint32_t rs, uint32_t jt, int nvalid, int tid) {
    using T = TileRegs<HD, FMT, NB, NT>;
    #pragma unroll
    for (int i = 0; i < T::KIT; i++) {
        const int it = i * NT + tid, key = it / T::NBLK, blk = it % T::NBLK;
        #pragma unroll
        for (int x = 0; x < T::W; x++) R.k[i][x] = 0;
        if (it < NB * T::NBLK && key < nvalid) load_item<FMT>(R.k[i], kb + (size_t) (jt + key) * rs, blk);
    }
    #pragma unroll
    for (int i = 0; i < T::VIT; i++) {
        const int it = i * NT + tid, kp = it / T::NBLK, blk = it % T::NBLK;
        #pragma unroll
        for (int x = 0; x < T::W; x++) R.v[i][0][x] = R.v[i][1][x] = 0;
        if (it < NB / 2 * T::NBLK) {
            if (2 * kp < nvalid) load_item<FMT>(R.v[i][0], vb + (size_t) (jt + 2 * kp) * rs, blk);
            if (2 * kp + 1 < nvalid) load_item<FMT>(R.v[i][1], vb + (size_t) (jt + 2 * kp + 1) * rs, blk);
        }
    }
}

// registers -> LDS: K as exact integer-valued fp16 + Ksc[blk][key] = d * s_mul; V transposed Vt[dim][key] = f16(d*q),
// written as (key pair) dwords. A zero-filled item (past nvalid) writes zeros and a zero scale.
template <int HD, int FMT, int NB, int NT>
__device__ __forceinline__ void store_tile(const TileRegs<HD, FMT, NB, NT> & R, _Float16 * __restrict__ Ks, float * __restrict__ Ksc,
                                           _Float16 * __restrict__ Vt, int tid, float s_mul) {
    using T = TileRegs<HD, FMT, NB, NT>;
    constexpr int KS = HD + 8, VS = NB + 4;
    #pragma unroll
    for (int i = 0; i < T::KIT; i++) {
        const int it = i * NT + tid, key = it / T::NBLK, blk = it % T::NBLK;
        if (it >= NB * T::NBLK) break;
        const uint32_t * w = R.k[i];
        pa_u4 o[4];
        float sc;
        if constexpr (FMT == 1) {
            sc = pa_f16_bits_to_f32((uint16_t) w[0]) * s_mul;
            #pragma unroll
            for (int q = 0; q < 8; q++) {
                uint32_t lo, hi;
                pa_int_q8x4(w[1 + q], lo, hi);
                o[q / 2][(q % 2) * 2 + 0] = lo;
                o[q / 2][(q % 2) * 2 + 1] = hi;
            }
        } else if constexpr (FMT == 2) {
            sc = pa_f16_bits_to_f32((uint16_t) w[0]) * s_mul;
            #pragma unroll
            for (int q = 0; q < 4; q++) {   // bytes 4q..4q+3: low nibbles = elements 4q.., high nibbles = 16 + 4q..
                uint32_t lo, hi;
                pa_int_nib4(w[1 + q] & 0x0f0f0f0fu, lo, hi);
                o[q / 2][(q % 2) * 2 + 0] = lo;
                o[q / 2][(q % 2) * 2 + 1] = hi;
                pa_int_nib4((w[1 + q] >> 4) & 0x0f0f0f0fu, lo, hi);
                o[2 + q / 2][(q % 2) * 2 + 0] = lo;
                o[2 + q / 2][(q % 2) * 2 + 1] = hi;
            }
        } else {
            sc = s_mul;
            #pragma unroll
            for (int c = 0; c < 4; c++) o[c] = (pa_u4){w[4 * c], w[4 * c + 1], w[4 * c + 2], w[4 * c + 3]};
        }
        pa_u4 * dst = (pa_u4 *) (Ks + key * KS + blk * 32);
        #pragma unroll
        for (int c = 0; c < 4; c++) dst[c] = o[c];
        Ksc[blk * NB + key] = sc;
    }
    #pragma unroll
    for (int i = 0; i < T::VIT; i++) {
        const int it = i * NT + tid, kp = it / T::NBLK, blk = it % T::NBLK, k0 = 2 * kp;
        if (it >= NB / 2 * T::NBLK) break;
        const uint32_t * a = R.v[i][0], * b = R.v[i][1];
        uint32_t * col = (uint32_t *) (Vt + (blk * 32) * VS + k0);   // dim blk*32 + d at col + d*VS/2
        if constexpr (FMT == 1) {
            const pa_h2 d2 = {__builtin_bit_cast(_Float16, (uint16_t) a[0]), __builtin_bit_cast(_Float16, (uint16_t) b[0])};
            const pa_h2 bias = {(_Float16) 1152.0f, (_Float16) 1152.0f};
            #pragma unroll
            for (int q = 0; q < 8; q++) {
                const uint32_t x0 = a[1 + q] ^ 0x80808080u, x1 = b[1 + q] ^ 0x80808080u;
                #pragma unroll
                for (int e = 0; e < 4; e++) col[(4 * q + e) * (VS / 2)] = pa_as_u32((pa_as_h2(pa_pair_byte(x1, x0, e)) - bias) * d2);
            }
        } else if constexpr (FMT == 2) {
            const pa_h2 d2 = {__builtin_bit_cast(_Float16, (uint16_t) a[0]), __builtin_bit_cast(_Float16, (uint16_t) b[0])};
            const pa_h2 bias = {(_Float16) 1032.0f, (_Float16) 1032.0f};
            #pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t l0 = a[1 + q] & 0x0f0f0f0fu, l1 = b[1 + q] & 0x0f0f0f0fu;
                const uint32_t h0 = (a[1 + q] >> 4) & 0x0f0f0f0fu, h1 = (b[1 + q] >> 4) & 0x0f0f0f0fu;
                #pragma unroll
                for (int e = 0; e < 4; e++) {
                    col[(4 * q + e) * (VS / 2)] = pa_as_u32((pa_as_h2(pa_pair_byte(l1, l0, e)) - bias) * d2);
                    col[(16 + 4 * q + e) * (VS / 2)] = pa_as_u32((pa_as_h2(pa_pair_byte(h1, h0, e)) - bias) * d2);
                }
            }
        } else {
            #pragma unroll
            for (int q = 0; q < 16; q++) {   // dword q = dims 2q, 2q+1
                col[(2 * q) * (VS / 2)] = pa_perm(b[q], a[q], 0x05040100u);
                col[(2 * q + 1) * (VS / 2)] = pa_perm(b[q], a[q], 0x07060302u);
            }
        }
    }
}

// ---------------------------------------------------------------- tiles of a chunk, page by page
struct TileIt {
    uint32_t p, jt, j1;   // page, first key of the tile in the page, end of the chunk's part of the page
    // from page p on: the first page that holds keys of [key_lo, key_hi), and its key range in page coordinates
    __device__ __forceinline__ void settle(const AttnArgs & a, uint32_t key_lo, uint32_t key_hi) {
        while (p < a.n_pages && (a.pstart[p + 1] <= key_lo || a.pstart[p + 1] == a.pstart[p])) p++;
        if (p < a.n_pages) {
            jt = max(key_lo, a.pstart[p]) - a.pstart[p];
            j1 = min(key_hi, a.pstart[p + 1]) - a.pstart[p];
        }
    }
    __device__ __forceinline__ bool valid(const AttnArgs & a, uint32_t key_hi) const { return p < a.n_pages && a.pstart[p] + jt < key_hi; }
};

// ---------------------------------------------------------------- the attention kernel
template <int HD, int FMT, int RT, int WR, int WK, int NB>
__global__ __launch_bounds__(64 * WR * WK) void attn_kernel(const AttnArgs a) {
    constexpr int NT = 64 * WR * WK;
    constexpr int KS = HD + 8, VS = NB + 4;
    constexpr int ND = HD / 16;        // 16-dim blocks of O^T
    constexpr int NKD = HD / 32;       // 32-dim blocks (= quant blocks) of QK
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

    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int wr = wave % WR, wk = wave / WR, g = lane / 16, n = lane % 16;
    const uint32_t row_base = rb * ROWS_WG + wr * RT * 16;   // first row of this wave's row tiles (within the head)

    // ---- start the first tile's loads, then prepare Q while they fly
    TileIt itr = {0, 0, 0};
    itr.settle(a, key_lo, key_hi);
    TileRegs<HD, FMT, NB, NT> R;
    bool have = itr.valid(a, key_hi);
    if (have) load_tile<HD, FMT, NB, NT>(R, a.kp[itr.p] + (size_t) h * a.hb, a.vp[itr.p] + (size_t) h * a.hb, a.rs, itr.jt,
                                         (int) min((uint32_t) NB, itr.j1 - itr.jt), tid);

    // Q^T fragments (B operand of QK): lane (g, n) holds row n, dims 32kd + 8g .. +7, as an fp16 hi + lo pair whose sum is
    // exactly the value the dot product must see. ggml mode with quantized K: q8_0 of each 32-block (d = amax/127,
    // id = 1/d, q = roundf(x*id), d -> fp16; quantize_row_q8_0_ref), value d16*q (exact in fp32), hi = f16, lo = f16(rest).
    // ggml mode with f16 K: f16(x) (ggml's vec_dot_type for f16). PA_QMODE_F16: f16(x*scale) (the reference engines).
    pa_h8 qh[RT][NKD], ql[RT][NKD];
    const bool qquant = a.qmode == 0 && FMT != 0;
    #pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const uint32_t row = row_base + rt * 16 + n;
        const bool live = row < a.rows;
        const float * qrow = a.q + ((size_t) h * a.rows + (live ? row : 0)) * HD + 8 * g;
        #pragma unroll
        for (int kd = 0; kd < NKD; kd++) {
            float x[8];
            const pa_f4 x0 = live ? *(const pa_f4 *) (qrow + 32 * kd) : (pa_f4){0.f, 0.f, 0.f, 0.f};
            const pa_f4 x1 = live ? *(const pa_f4 *) (qrow + 32 * kd + 4) : (pa_f4){0.f, 0.f, 0.f, 0.f};
            x[0] = x0[0]; x[1] = x0[1]; x[2] = x0[2]; x[3] = x0[3]; x[4] = x1[0]; x[5] = x1[1]; x[6] = x1[2]; x[7] = x1[3];
            if (qquant) {
                float am = 0.0f;
                #pragma unroll
                for (int j = 0; j < 8; j++) am = fmaxf(am, fabsf(x[j]));
                am = pa_wave_max16x4(am);                              // the block's 32 values sit in lanes n, n+16, n+32, n+48
                const float d = am / 127.0f;
                const float id = d != 0.0f ? 1.0f / d : 0.0f;
                const float d16 = (float) (_Float16) d;
                #pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float t = d16 * roundf(x[j] * id);
                    const _Float16 th = (_Float16) t;
                    qh[rt][kd][j] = th;
                    ql[rt][kd][j] = (_Float16) (t - (float) th);
                }
            } else {
                const float mul = a.qmode == 0 ? 1.0f : a.scale;
                #pragma unroll
                for (int j = 0; j < 8; j++) { qh[rt][kd][j] = (_Float16) pa_f32(x[j] * mul); ql[rt][kd][j] = (_Float16) 0.0f; }
            }
        }
    }
    pa_f4 o[RT][ND];
    float mref[RT], mtrue[RT], lrow[RT];
    #pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        mref[rt] = mtrue[rt] = -INFINITY; lrow[rt] = 0.0f;
        #pragma unroll
        for (int d = 0; d < ND; d++) o[rt][d] = (pa_f4){0.f, 0.f, 0.f, 0.f};
    }
    const float s_mul = a.s_mul;

    while (have) {
        const int nvalid = (int) min((uint32_t) NB, itr.j1 - itr.jt);
        const bool full = nvalid == NB;
        __syncthreads();                                             // the previous tile's readers are done
        store_tile<HD, FMT, NB, NT>(R, Ks, Ksc, Vt, tid, s_mul);
        // next tile: its bytes fly while this one is computed
        itr.jt += NB;
        if (itr.jt >= itr.j1) { itr.p++; itr.settle(a, key_lo, key_hi); }
        have = itr.valid(a, key_hi);
        if (have) load_tile<HD, FMT, NB, NT>(R, a.kp[itr.p] + (size_t) h * a.hb, a.vp[itr.p] + (size_t) h * a.hb, a.rs, itr.jt,
                                             (int) min((uint32_t) NB, itr.j1 - itr.jt), tid);
        __syncthreads();
        #pragma unroll
        for (int ks = 0; ks < KPW / 32; ks++) {
            const int kbase = wk * KPW + ks * 32;                 // first key of this 32-key step within the tile
            if (kbase >= nvalid) break;
            // S^T = K . Q^T for two 16-key subtiles, one MFMA (two with the lo half) per 32-dim block: exact partial dots,
            // combined in fp32 with the block's K scale (already times s_mul: base-2 logits come out)
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
                    if (qquant) {
                        a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, ql[rt][kd], a0, 0, 0, 0);
                        a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, ql[rt][kd], a1, 0, 0, 0);
                    }
                    s[rt][0] += d0 * a0;
                    s[rt][1] += d1 * a1;
                }
            }
            pa_h8 pf[RT];
            #pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                float v[8];
                #pragma unroll
                for (int i = 0; i < 4; i++) { v[i] = s[rt][0][i]; v[4 + i] = s[rt][1][i]; }
                if (!full) {
                    #pragma unroll
                    for (int i = 0; i < 4; i++) {
                        if (kbase + 4 * g + i >= nvalid) v[i] = -INFINITY;
                        if (kbase + 16 + 4 * g + i >= nvalid) v[4 + i] = -INFINITY;
                    }
                }
                float tm = v[0];
                #pragma unroll
                for (int i = 1; i < 8; i++) tm = fmaxf(tm, v[i]);
                tm = pa_wave_max16x4(tm);
                mtrue[rt] = fmaxf(mtrue[rt], tm);
                // the probabilities use a reference max that moves only when a score exceeds it by more than 2^8, so the
                // O rescale runs rarely; p <= 256 stays well inside fp16. The exact max is kept in mtrue.
                const bool need = tm > mref[rt] + 8.0f;
                if (__any(need)) {
                    const float nr = need ? mtrue[rt] : mref[rt];
                    const float alpha = mref[rt] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mref[rt] - nr);
                    lrow[rt] *= alpha;
                    #pragma unroll
                    for (int d = 0; d < ND; d++) o[rt][d] *= alpha;
                    mref[rt] = nr;
                }
                const float ms = mref[rt] == -INFINITY ? 0.0f : mref[rt];
                float sum = 0.0f;
                #pragma unroll
                for (int i = 0; i < 8; i++) { v[i] = __builtin_amdgcn_exp2f(v[i] - ms); sum += v[i]; }
                lrow[rt] += sum;
                #pragma unroll
                for (int i = 0; i < 8; i++) pf[rt][i] = (_Float16) v[i];
            }
            // O^T += V^T . P^T: lane (g, n) = dim 16*db + n, keys kbase + 4g..+3 and kbase + 16 + 4g..+3
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

    // ---- per-row sums over the 4 lane groups; rebase (O, l) from the reference max to the exact max
    float mrow[RT];
    #pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        lrow[rt] = pa_wave_sum16x4(lrow[rt]);
        const float f = mref[rt] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mref[rt] - mtrue[rt]);
        if (__any(f != 1.0f)) {
            lrow[rt] *= f;
            #pragma unroll
            for (int d = 0; d < ND; d++) o[rt][d] *= f;
        }
        mrow[rt] = mtrue[rt];
    }

    // ---- this workgroup's result: final (one chunk) or a split-K slot
    const bool direct = a.n_chunks == 1 && a.fused;
    const uint32_t slot = a.slot0 + c;
    float * po = a.po + ((size_t) slot * a.nkv + h) * a.qr * HD;
    float2 * pml = a.pml + ((size_t) slot * a.nkv + h) * a.qr;
    float * fO = a.O + (size_t) h * a.rows * HD;
    float * fm = a.m + (size_t) h * a.rows, * fl = a.l + (size_t) h * a.rows;
    auto emit = [&](uint32_t row, int d4, pa_f4 val, float M, float L) {
        if (direct) {
            *(pa_f4 *) (fO + (size_t) row * HD + 4 * d4) = val;
            if (d4 == 0) { fm[row] = M == -INFINITY ? -INFINITY : M * PA_LN2; fl[row] = L; }
        } else {
            *(pa_f4 *) (po + (size_t) row * HD + 4 * d4) = val;
            if (d4 == 0) pml[row] = make_float2(M, L);
        }
    };
    if constexpr (WK == 1) {
        #pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const uint32_t row = row_base + rt * 16 + n;
            if (row >= a.rows) continue;
            #pragma unroll
            for (int db = 0; db < ND; db++) emit(row, 4 * db + g, o[rt][db], mrow[rt], lrow[rt]);
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
            for (int q = 0; q < WK; q++) M = fmaxf(M, cML[q * ROWS_WG + lr].x);
            const float Ms = M == -INFINITY ? 0.0f : M;
            pa_f4 acc = {0.f, 0.f, 0.f, 0.f};
            float L = 0.0f;
            #pragma unroll
            for (int q = 0; q < WK; q++) {
                const float2 ml = cML[q * ROWS_WG + lr];
                const float wt = __builtin_amdgcn_exp2f(ml.x - Ms);
                L += wt * ml.y;
                acc += wt * *(const pa_f4 *) (cO + ((size_t) q * ROWS_WG + lr) * HD + 4 * d4);
            }
            emit(row, d4, acc, M, L);
        }
    }
}

// ---------------------------------------------------------------- split-K fold as its own kernel
// The reply format of a merged row (the ATTN reply, phone-attn.h:651-655), written in place of (O, m, l) when the call
// asks for it: Oh = f16(O * (1 / L)) (0 where L = 0) for k consecutive dims, lse = M ln 2 + log L by the thread given
// `row_stats`. The same roundings as storing (O, m, l) and normalising them afterwards.
template <int K>
__device__ __forceinline__ void merge_write_reply(const MergeArgs & a, size_t off, const float * o, float M, float L, uint32_t r,
                                                  bool row_stats) {
    #pragma clang fp contract(off)
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    #pragma unroll
    for (int k = 0; k < K; k++) a.Oh[off + k] = __builtin_bit_cast(uint16_t, (_Float16) pa_f32(o[k] * inv));
    if (row_stats) {
        const float mm = M == -INFINITY ? -INFINITY : M * PA_LN2;
        a.lse[r] = L > 0.0f ? mm + logf(L) : -INFINITY;
    }
}

// Used when one call needs several attention launches (more than MAXP pages). One workgroup per output row; thread t
// folds dims 4*(t % (HD/4)) over slots t / (HD/4), t / (HD/4) + SG, ...
template <int HD>
__global__ __launch_bounds__(256) void merge_kernel(const MergeArgs a) {
    constexpr int TPR = HD / 4, SG = 256 / TPR;
    __shared__ pa_f4 red[SG][TPR];
    __shared__ float redl[SG];
    __shared__ float redm[256];
    const uint32_t r = blockIdx.x;                   // output row = h*rows + i
    const uint32_t h = r / a.rows, i = r % a.rows;
    const int t = threadIdx.x, d4 = t % TPR, sg = t / TPR;
    const size_t pr = ((size_t) h * a.qr + i) * a.rst;              // slot s at s * a.sst + pr
    float M = -INFINITY;
    for (uint32_t s = t; s < a.n_slots; s += 256) M = fmaxf(M, a.pml[s * a.sst + pr].x);
    redm[t] = M;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
        if (t < off) redm[t] = fmaxf(redm[t], redm[t + off]);
        __syncthreads();
    }
    M = redm[0];
    const float Ms = M == -INFINITY ? 0.0f : M;
    pa_f4 acc = {0.f, 0.f, 0.f, 0.f};
    float L = 0.0f;
    for (uint32_t s = sg; s < a.n_slots; s += SG) {
        const float2 ml = a.pml[s * a.sst + pr];
        const float w = __builtin_amdgcn_exp2f(ml.x - Ms);   // ml.x = -inf -> 0 (an empty slot)
        L += w * ml.y;
        acc += w * *(const pa_f4 *) (a.po + (s * a.sst + pr) * HD + 4 * d4);
    }
    red[sg][d4] = acc;
    if (d4 == 0) redl[sg] = L;
    __syncthreads();
    if (sg == 0) {
        for (int q = 1; q < SG; q++) acc += red[q][d4];
        for (int q = 1; q < SG; q++) L += redl[q];                    // every thread: the reply needs L
        if (a.Oh) {
            const float ov[4] = {acc[0], acc[1], acc[2], acc[3]};
            merge_write_reply<4>(a, (size_t) r * HD + 4 * d4, ov, M, L, r, d4 == 0);
            return;
        }
        *(pa_f4 *) (a.O + (size_t) r * HD + 4 * d4) = acc;
        if (d4 == 0) { a.m[r] = M == -INFINITY ? -INFINITY : M * PA_LN2; a.l[r] = L; }
    }
}

// Many slots (split-K decode up to 256, verify up to 64): one workgroup of NT threads (256, or one wave for at most 64
// slots) per (row, 32 dims), every load of the fold issued at once (one memory latency, not one per slot). Lane l of
// wave v reads dims 4 (l % 8) .. +3 of slots 64 v + l / 8 + 8 j (j < 8), so that eight lanes read one slot's 128 bytes
// and a load instruction touches eight whole lines; thread t also reads slot t's (max, sum). The weights reach the
// lanes that hold a slot's dims by a shuffle, the dims' sums by xor-shuffles over the eight-lane groups, then across
// waves through LDS.
template <int HD, int NT>
__global__ __launch_bounds__(NT) void merge_wide_kernel(const MergeArgs a) {
    constexpr int NQ = HD / 32, NWV = NT / 64;
    __shared__ float sM[NWV], sL[NWV];
    __shared__ pa_f4 sA[NWV][8];
    const uint32_t r = blockIdx.x / NQ, dq = blockIdx.x % NQ;   // output row h*rows + i, dims 32 dq .. +31
    const uint32_t h = r / a.rows, i = r % a.rows;
    const int t = threadIdx.x, lane = t % 64, wv = t / 64;
    const size_t pr = ((size_t) h * a.qr + i) * a.rst;              // slot s of the row at s * a.sst + pr
    pa_f4 o[8];
    #pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t s = 64 * wv + lane / 8 + 8 * j;
        o[j] = s < a.n_slots ? *(const pa_f4 *) (a.po + (s * a.sst + pr) * HD + 32 * dq + 4 * (lane % 8))
                             : (pa_f4){0.f, 0.f, 0.f, 0.f};
    }
    const float2 ml = (uint32_t) t < a.n_slots ? a.pml[t * a.sst + pr] : make_float2(-INFINITY, 0.0f);
    float M = ml.x;
    #pragma unroll
    for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
    if constexpr (NWV > 1) {
        if (lane == 0) sM[wv] = M;
        __syncthreads();
        #pragma unroll
        for (int k = 0; k < NWV; k++) M = fmaxf(M, sM[k]);
    }
    const float Ms = M == -INFINITY ? 0.0f : M;
    const float w = __builtin_amdgcn_exp2f(ml.x - Ms);              // -inf (an empty or absent slot) -> 0
    float L = w * ml.y;
    #pragma unroll
    for (int off = 32; off > 0; off >>= 1) L += __shfl_xor(L, off);
    pa_f4 acc = {0.f, 0.f, 0.f, 0.f};
    #pragma unroll
    for (int j = 0; j < 8; j++) acc += __shfl(w, lane / 8 + 8 * j) * o[j];   // slot 64 wv + l / 8 + 8 j is this wave's lane l / 8 + 8 j
    #pragma unroll
    for (int off = 8; off < 64; off <<= 1)
        #pragma unroll
        for (int k = 0; k < 4; k++) acc[k] += __shfl_xor(acc[k], off);
    if constexpr (NWV > 1) {
        if (lane < 8) sA[wv][lane] = acc;
        if (lane == 0) sL[wv] = L;
        __syncthreads();
        if (wv != 0 || lane >= 8) return;
        acc = sA[0][lane];
        L = sL[0];
        #pragma unroll
        for (int k = 1; k < NWV; k++) { acc += sA[k][lane]; L += sL[k]; }
    } else if (lane >= 8) {
        return;
    }
    // lanes 0-7 of wave 0: dims 32 dq + 4 lane .. +3
    const size_t off = (size_t) r * HD + 32 * dq + 4 * lane;
    if (a.Oh) {
        const float v[4] = {acc[0], acc[1], acc[2], acc[3]};
        merge_write_reply<4>(a, off, v, M, L, r, dq == 0 && lane == 0);
        return;
    }
    *(pa_f4 *) (a.O + off) = acc;
    if (dq == 0 && lane == 0) {
        a.m[r] = M == -INFINITY ? -INFINITY : M * PA_LN2;
        a.l[r] = L;
    }
}

// Few slots (prefill, up to 16): 256 / (HD / 4) rows per workgroup, HD / 4 threads per row (4 dims each), every
// slot's load issued at once.
template <int HD>
__global__ __launch_bounds__(256) void merge_rows_kernel(const MergeArgs a) {
    constexpr int TPR = HD / 4, RPW = 256 / TPR, MS = 16;
    const int t = threadIdx.x, d4 = t % TPR;
    const uint32_t r = blockIdx.x * RPW + t / TPR;                   // output row h*rows + i
    if (r >= a.nkv * a.rows) return;
    const uint32_t h = r / a.rows, i = r % a.rows;
    const size_t pr = ((size_t) h * a.qr + i) * a.rst;              // slot s at s * a.sst + pr
    float2 ml[MS];
    pa_f4 o[MS];
    #pragma unroll
    for (int s = 0; s < MS; s++) {
        if ((uint32_t) s < a.n_slots) {
            ml[s] = a.pml[s * a.sst + pr];
            o[s] = *(const pa_f4 *) (a.po + (s * a.sst + pr) * HD + 4 * d4);
        } else {
            ml[s] = make_float2(-INFINITY, 0.0f);
            o[s] = (pa_f4){0.f, 0.f, 0.f, 0.f};
        }
    }
    float M = -INFINITY;
    #pragma unroll
    for (int s = 0; s < MS; s++) M = fmaxf(M, ml[s].x);
    const float Ms = M == -INFINITY ? 0.0f : M;
    pa_f4 acc = {0.f, 0.f, 0.f, 0.f};
    float L = 0.0f;
    #pragma unroll
    for (int s = 0; s < MS; s++) {
        const float w = __builtin_amdgcn_exp2f(ml[s].x - Ms);       // -inf (an empty or absent slot) -> 0
        acc += w * o[s];
        L += w * ml[s].y;
    }
    if (a.Oh) {
        const float ov[4] = {acc[0], acc[1], acc[2], acc[3]};
        merge_write_reply<4>(a, (size_t) r * HD + 4 * d4, ov, M, L, r, d4 == 0);
        return;
    }
    *(pa_f4 *) (a.O + (size_t) r * HD + 4 * d4) = acc;
    if (d4 == 0) { a.m[r] = M == -INFINITY ? -INFINITY : M * PA_LN2; a.l[r] = L; }
}

// ---------------------------------------------------------------- launch table
template <int HD, int FMT, int RT, int WR, int WK, int NB>
static hipError_t launch_attn(const AttnArgs & a, uint32_t grid, hipStream_t st) {
    hipLaunchKernelGGL((attn_kernel<HD, FMT, RT, WR, WK, NB>), dim3(grid), dim3(64 * WR * WK), 0, st, a);
    return hipGetLastError();
}

// configurations (RT, WR, WK, NB) at head dim 256: decode-shaped calls (<= 16 rows per KV head) split each 128-key
// tile over 4 waves (16 rows, one workgroup per CU by LDS); more rows take 64 rows per workgroup (registers).
template <int FMT>
static hipError_t launch_attn_cfg(int cfg, const AttnArgs & a, uint32_t grid, hipStream_t st) {
    if (cfg == CFG_DECODE) return launch_attn<256, FMT, 1, 1, 4, 128>(a, grid, st);
    return launch_attn<256, FMT, 1, 4, 1, 64>(a, grid, st);
}

hipError_t launch_attention(int hd, int fmt, int cfg, const AttnArgs & a, uint32_t grid, hipStream_t st) {
    if (hd != 256) return hipErrorInvalidValue;
    if (fmt == 0) return launch_attn_cfg<0>(cfg, a, grid, st);
    if (fmt == 1) return launch_attn_cfg<1>(cfg, a, grid, st);
    if (fmt == 2) return launch_attn_cfg<2>(cfg, a, grid, st);
    return hipErrorInvalidValue;
}

void cfg_geometry(int cfg, int & rows_per_wg, int & nb) {
    if (cfg == CFG_DECODE) { rows_per_wg = 16; nb = 128; }
    else { rows_per_wg = 64; nb = 64; }
}

hipError_t launch_merge(int hd, const MergeArgs & a, hipStream_t st) {
    const uint32_t grid = a.nkv * a.rows;
    if (a.n_slots > 16 && a.n_slots <= 64) {                        // many slots: one thread per slot, one wave
        if (hd == 128) hipLaunchKernelGGL((merge_wide_kernel<128, 64>), dim3(grid * 4), dim3(64), 0, st, a);
        else if (hd == 256) hipLaunchKernelGGL((merge_wide_kernel<256, 64>), dim3(grid * 8), dim3(64), 0, st, a);
        else return hipErrorInvalidValue;
        return hipGetLastError();
    }
    if (a.n_slots > 64 && a.n_slots <= 256) {                       // up to 256: four waves
        if (hd == 128) hipLaunchKernelGGL((merge_wide_kernel<128, 256>), dim3(grid * 4), dim3(256), 0, st, a);
        else if (hd == 256) hipLaunchKernelGGL((merge_wide_kernel<256, 256>), dim3(grid * 8), dim3(256), 0, st, a);
        else return hipErrorInvalidValue;
        return hipGetLastError();
    }
    if (a.n_slots <= 16) {                                           // few slots: several rows per workgroup
        if (hd == 128) hipLaunchKernelGGL(merge_rows_kernel<128>, dim3((grid + 7) / 8), dim3(256), 0, st, a);
        else if (hd == 256) hipLaunchKernelGGL(merge_rows_kernel<256>, dim3((grid + 3) / 4), dim3(256), 0, st, a);
        else return hipErrorInvalidValue;
        return hipGetLastError();
    }
    if (hd == 128) hipLaunchKernelGGL(merge_kernel<128>, dim3(grid), dim3(256), 0, st, a);
    else if (hd == 256) hipLaunchKernelGGL(merge_kernel<256>, dim3(grid), dim3(256), 0, st, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace pa_hip
