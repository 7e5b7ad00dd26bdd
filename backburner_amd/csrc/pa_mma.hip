// pa_mma.hip - partial attention for many query rows per KV head (16-token verify, 512-token prefill chunks, and any
// shape with more than 8 rows) over q8_0 / q4_0 / f16 K and V, head dim 128, fp16 matrix cores (gfx950).
//
// One workgroup = one KV head x one block of 32*NW query rows x one chunk of consecutive 32-key tiles; NW waves, 32
// rows each. Per tile the workgroup dequantizes V once into LDS as fp16 (d*q rounded once: the quants become fp16
// integers exactly through the 0x64 exponent byte, then one subtract and one multiply), and K too unless the call takes
// the exact block dots (EX below, which keep K's raw quants), double-buffered, with the next tile's raw bytes already in
// flight into registers. Each wave then computes, with v_mfma_f32_32x32x16_f16,
//   S^T (32 keys x 32 rows) = K . Q'^T      (8 MFMAs over the 128 dims; Q' stays in registers for the whole kernel),
// so lane (h, n) holds row n's scores of keys 8j + 4h + i (j, i < 4) - which is exactly the B operand layout of
//   O^T (128 dims x 32 rows) += V^T . P^T    (4 dim blocks x 2 MFMAs; V^T read from LDS by ds_read_b64_tr_b16),
// so the probabilities never leave registers, and every value a lane holds belongs to its own row n: the running max
// and sum need one exchange with lane n + 32 per tile and no LDS.
//
// Q' is the query as fp16: PA_QMODE_F16 takes fp16(q*scale) (the reference engines' Qs, phone-attn.h:595-599), and f16
// K in PA_QMODE_GGML fp16(q), K's vec_dot type in ggml's CPU flash_attn_ext (the scale then multiplies the score).
// Quantized K in PA_QMODE_GGML takes exact block dots instead (EX below): Q converted to q8_0 per 32-block as ggml does
// (quantize_row_q8_0_ref), K staged as its raw quants, one int8 MFMA per 32-dim block, and ggml's per-block scaling in
// fp32. Online softmax in base 2 with a reference max that moves only when a score exceeds it by more than 2^MM_PMAX (O is rescaled
// rarely); the exact max is tracked beside it and applied at the end. The row sum adds the fp16 probabilities the PV
// MFMAs consume. Output: one split-K slot per workgroup (O unnormalised against the base-2 max, max, sum), folded by
// the merge kernels, or the final (O, m, l) when the call has a single chunk.
//
// Reference roles: pa_attn_big + pa_big_load (pa-metal.mm:379-487: per (row tile, KV head, key chunk) dequantize a
// K/V block into threadgroup memory as half, S = QK^T on the matrix units, online softmax with key masking, O = a O +
// PV, write a slot); ggml's q8_0 query conversion (restated in oracle/pa_oracle.c, orc_attn_ggml).
#include "pa_mma.h"
#include <hip/hip_ext.h>

namespace pa_hip {

constexpr int MM_HD = 128;
constexpr int MM_KST = 2 * MM_HD + 16;            // K tile row stride (bytes): 16 consecutive keys' 16-byte reads hit
                                                  // distinct banks
constexpr int MM_VST = 2 * MM_HD + 64;            // V tile row stride: the 4 rows x 64 bytes of a half-wave's
                                                  // transposing reads hit distinct banks
constexpr int MM_KT = 32 * MM_KST, MM_VT = 32 * MM_VST;
constexpr int MM_KST8 = MM_HD + 16;               // raw K tile row stride (EX): 16 consecutive keys' 16-byte
                                                  // reads hit distinct banks
constexpr int MM_KSC = 32 * 8;                    // exact-QK kernels: the tile's K block scales, [key][4 blocks] fp16
constexpr int MM_STAGE = MM_KT + MM_VT + MM_KSC;

// The query rows as the fp16 B operand (lane (h2, n) holds row n, dims 16kk + 8h2 + t): f16(q * scale), or f16(q) for
// f16 K in PA_QMODE_GGML (ggml's f16 vec_dot type)
__device__ __forceinline__ void mm_prep_q(const AttnArgs & a, uint32_t h, uint32_t row, bool rlive, int h2, mm_h8 (&Qf)[8]) {
    const float * qrow = a.q + ((size_t) h * a.rows + (rlive ? row : 0)) * MM_HD + 8 * h2;
    const uint32_t qmask = rlive ? 0xffffffffu : 0u;
    const float qs = a.qmode == 0 ? 1.0f : a.scale;
    #pragma unroll
    for (int kk = 0; kk < 8; kk++) {
        const pa_f4 x0 = __builtin_bit_cast(pa_f4, __builtin_bit_cast(pa_u4, *(const pa_f4 *) (qrow + 16 * kk)) & qmask);
        const pa_f4 x1 = __builtin_bit_cast(pa_f4, __builtin_bit_cast(pa_u4, *(const pa_f4 *) (qrow + 16 * kk + 4)) & qmask);
        mm_h8 f;
        #pragma unroll
        for (int t = 0; t < 8; t++) f[t] = (_Float16) pa_f32((t < 4 ? x0[t] : x1[t - 4]) * qs);   // f2h(q * scale)
        Qf[kk] = f;
    }
}

// The query rows as the int8 B operand of the exact block dots (EX): lane (h2, n) holds row n's ggml q8_0 quants of
// dims 32b + 16h2 .. +15 (quantize_row_q8_0_ref: d = amax / 127, id = 1 / d, q = roundf(x * id), d stored as fp16),
// and per block b the (hi, lo) fp16 pair whose
// sum is the fp16 block scale times scale * log2 e (dqb[b], hi in the low half): to about 22 bits where that product
// is at least 2^-9; below, lo falls into the fp16 subnormals and the pair keeps an absolute error of at most 2^-25, so
// the block's term dot_b * dk_b * (hi + lo) errs by at most |dot_b| * dk_b * 2^-25 in base-2 units.
// For q4_0 K (unsigned nibbles u = q + 8 in the int8 MFMA) it also gives, per block, the (hi, lo) pair of
// -8 * (sum of the row's block quants) * (hi + lo) in fp32 (dcb[b]): the offset the unsigned nibbles add to each block
// dot, times the row's scale pair; a key's block scale times it is that block's correction of the score.
template <int FMT>
__device__ __forceinline__ void mm_prep_qi8(const AttnArgs & a, uint32_t h, uint32_t row, bool rlive, int h2, pa_u4 (&Qi)[4],
                                            uint32_t (&dqb)[4], uint32_t (&dcb)[4]) {
    const float * qrow = a.q + ((size_t) h * a.rows + (rlive ? row : 0)) * MM_HD + 16 * h2;
    const uint32_t qmask = rlive ? 0xffffffffu : 0u;
    const float scale = a.scale;
    #pragma unroll
    for (int b = 0; b < 4; b++) {
        #pragma clang fp contract(off)
        pa_f4 x[4];
        #pragma unroll
        for (int j = 0; j < 4; j++) x[j] = __builtin_bit_cast(pa_f4, __builtin_bit_cast(pa_u4, *(const pa_f4 *) (qrow + 32 * b + 4 * j)) & qmask);
        float am = 0.0f;
        #pragma unroll
        for (int j = 0; j < 4; j++) am = fmaxf(am, fmaxf(fmaxf(fabsf(x[j][0]), fabsf(x[j][1])), fmaxf(fabsf(x[j][2]), fabsf(x[j][3]))));
        am = mm_max32(am);                                           // the block's other 16 values: lane ^ 32
        const float d = am / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const float dq = (float) (_Float16) d * (scale * MM_LOG2E);   // the fp16 block scale * scale, base-2 units
        const _Float16 hi = (_Float16) dq, lo = (_Float16) (dq - (float) hi);
        dqb[b] = (uint32_t) __builtin_bit_cast(uint16_t, hi) | ((uint32_t) __builtin_bit_cast(uint16_t, lo) << 16);
        uint32_t w[4];
        int qs = 0;
        #pragma unroll
        for (int j = 0; j < 4; j++) {
            uint32_t v = 0;
            #pragma unroll
            for (int e = 0; e < 4; e++) {
                const int q = (int) roundf(x[j][e] * id);
                qs += q;
                v |= ((uint32_t) q & 0xffu) << (8 * e);
            }
            w[j] = v;
        }
        Qi[b] = (pa_u4){w[0], w[1], w[2], w[3]};
        if constexpr (FMT == 2) {
            const auto t = __builtin_amdgcn_permlane32_swap((unsigned) qs, (unsigned) qs, false, false);
            const int qsum = (int) t[0] + (int) t[1];                // the block's 32 quants: lanes l and l ^ 32
            const float c = (float) (-8 * qsum) * ((float) hi + (float) lo);
            const _Float16 chi = (_Float16) c, clo = (_Float16) (c - (float) chi);
            dcb[b] = (uint32_t) __builtin_bit_cast(uint16_t, chi) | ((uint32_t) __builtin_bit_cast(uint16_t, clo) << 16);
        }
    }
}

// Row n's result: the sum over both lanes, O rebased from the reference max to the exact one; the final (O, m, l)
// for a single-chunk call, else split-K slot c
__device__ __forceinline__ void mm_write_out(const AttnArgs & a, const mm_f16 (&O)[4], float mref, float mx, float lsum,
                                             uint32_t h, uint32_t row, bool rlive, int h2, uint32_t c) {
    const float lt = mm_sum32(lsum);
    const float f = mref == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mref - mx);
    if (!rlive) return;
    const bool direct = a.n_chunks == 1 && a.fused;
    float * dst = direct ? a.O + ((size_t) h * a.rows + row) * MM_HD
                         : a.po + (((size_t) h * a.qr + row) * a.slots + a.slot0 + c) * MM_HD;
    #pragma unroll
    for (int db = 0; db < 4; db++)
        #pragma unroll
        for (int j = 0; j < 4; j++) {
            const pa_f4 v = {O[db][4 * j] * f, O[db][4 * j + 1] * f, O[db][4 * j + 2] * f, O[db][4 * j + 3] * f};
            *(pa_f4 *) (dst + 32 * db + 8 * j + 4 * h2) = v;
        }
    if (h2 == 0) {
        if (direct) {
            a.m[(size_t) h * a.rows + row] = mx == -INFINITY ? -INFINITY : mx * PA_LN2;
            a.l[(size_t) h * a.rows + row] = lt * f;
        } else {
            a.pml[((size_t) h * a.qr + row) * a.slots + a.slot0 + c] = make_float2(mx, lt * f);
        }
    }
}

// EX: exact block dots, as ggml computes them (PA_QMODE_GGML over quantized K). K is staged as its raw quants, with the
// tile's fp16 block scales beside it (q8_0: the int8 quants as they are, half the LDS bytes of the fp16 tile; q4_0: the
// nibbles of one block half as unsigned bytes u = q + 8), and Q as ggml's q8_0 int8 quants. Per 32-block b one
// v_mfma_i32_32x32x32_i8 gives the integer dot itself (|dot| < 2^21), converted to fp32 exactly, and one fp16 MFMA the
// scale product dk_b(key) * (hi + lo)(row): dk_b at k = 0 and 1 of A, the row's pair at k = 0 and 1 of B (an outer
// product in otherwise zero operands). The scores are the fp32 sum over the blocks of dot_b * (scale product), started
// at -mref: ggml's per-block vec_dot arithmetic (vec_dot_q8_0_q8_0 / q4_0_q8_0), with the softmax scale and the base-2
// conversion inside each block's factor instead of the dot of two fp16-rounded operands. For q4_0 the start value also
// takes the offset of the unsigned nibbles, sum_b dk_b * (-8 * qsum_b) * (hi + lo)_b, from one more MFMA per tile.
// Otherwise (PA_QMODE_F16, f16 K) the QK is one fp16 rounding of each operand and each score is scaled and shifted by
// one fma.
// SKIP: a wave whose 32 rows are all past the call's rows only stages (its share of every tile's loads, dequant and LDS
// stores, and the barriers). For calls with one row block narrower than 32 * NW rows. Without SKIP there is no branch
// there: one costs 13-20 % on full row blocks, as it separates the next tile's loads from the QK MFMAs, which the
// compiler otherwise schedules in one basic block.
template <int FMT, int NW, bool SKIP, bool EX>
__global__ __launch_bounds__(64 * NW, 8 / NW) void mma_kernel(const AttnArgs a) {   // 2 waves per SIMD
    static_assert(!EX || FMT != 0, "the exact block dots take quantized K");
    constexpr int PF = 2;                                            // tiles whose raw bytes are in flight
    constexpr int NT = 64 * NW;
    constexpr int UPT = 512 / NT;                                    // staging units per thread (512 per tile)
    static_assert(UPT * NT == 512, "NW must be 4 or 8");
    __shared__ __attribute__((aligned(16))) char smem[2 * MM_STAGE];

    // ---- which (chunk, KV head, row block): row blocks fastest, so the workgroups that share a chunk's K/V run side
    // by side on one XCD (= blockIdx % 8 in dispatch order, which takes a contiguous item range) and share its L2
    const uint32_t bid = blockIdx.x, xcd = bid % 8, local = bid / 8;
    const uint32_t t8 = (a.n_items + 7) / 8;
    const uint32_t w = xcd * t8 + local;
    if (local >= t8 || w >= a.n_items) return;
    const uint32_t rb = w % a.nrb, h = (w / a.nrb) % a.nkv, c = w / (a.nrb * a.nkv);
    const uint32_t T = a.cstart[a.n_pages];                          // 32-key tiles of the call
    const uint32_t t0 = c * a.chunk, ntiles = min(t0 + a.chunk, T) - t0;   // this chunk's tiles [t0, t0 + ntiles)

    const int tid = threadIdx.x, lane = tid % 64;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const int n = lane & 31, h2 = lane >> 5;
    const uint32_t row = rb * (32 * NW) + 32 * wave + n;             // this lane's query row (within the KV head)
    const bool rlive = row < a.rows;
    const bool wlive = !SKIP || rb * (32 * NW) + 32 * wave < a.rows;    // uniform: the wave has a live row

    MmCursor cl, cc;                                                 // the next tile to load / to compute
    cl.init(a); cc.init(a);

    // ---- staging units of this thread: u = tid + NT*i -> tensor u >> 8 (= (wave + NW*i) >> 2, uniform), key
    // (u >> 3) & 31, block (u >> 1) & 3, half u & 1; rows past the page's end reload its last row (masked later)
    using F = MmFmt<FMT>;
    MmRaw<FMT> R0[UPT], R1[UPT];                                     // tile t's raw bytes in R(t % 2)
    // buffer loads: the tile's first row of this head as the scalar base, its rows up to the page's end as the range.
    // Past the chunk's last tile (live false) the same loads go out with an empty range (no memory access, zeros), so
    // that every step issues the same batch and the wait before a tile's dequant covers its own batch only.
    auto load_tile = [&](MmRaw<FMT> (&R)[UPT], uint32_t tau, bool live) {
        if (live) cl.seek(a, tau);
        const uint32_t j0 = live ? 32 * (tau - cl.tb) : 0u;
        const uint32_t last = live ? cl.nk - 1 - j0 : 0u;
        // the range covers the tile's rows only (at most 32 of rs bytes, rs < 2^26 by the host's check), so a page of
        // any size keeps the 32-bit byte count exact
        const uint32_t nrec = live ? min(last + 1, 32u) * a.rs : 0u;
        #pragma unroll
        for (int i = 0; i < UPT; i++) {
            const int u = tid + NT * i;
            const int tensor = (wave + NW * i) >> 2, key = (u >> 3) & 31, blk = (u >> 1) & 3, half = u & 1;
            const uint8_t * base = (tensor ? cl.vb : cl.kb) + (size_t) h * a.hb + (size_t) j0 * a.rs;
            const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc((void *) base, (short) 0, (int) nrec, 0x00020000);
            mm_load_unit_buf<FMT>(R[i], rsrc, min((uint32_t) key, last) * a.rs + blk * F::BB, half);
        }
    };
    auto store_tile = [&](const MmRaw<FMT> (&R)[UPT], int stage) {
        char * st = smem + stage * MM_STAGE;
        #pragma unroll
        for (int i = 0; i < UPT; i++) {
            const int u = tid + NT * i;
            const int tensor = (wave + NW * i) >> 2, key = (u >> 3) & 31, blk = (u >> 1) & 3, half = u & 1;
            pa_u4 lo, hi;
            if (EX && tensor == 0) {                                 // K: the raw int8 quants (q4_0: this half's
                                                                     // nibbles as unsigned bytes), the block scale beside
                if (half == 0) *(uint16_t *) (st + MM_KT + MM_VT + 8 * key + 2 * blk) = (uint16_t) R[i].d;
                pa_u4 q = R[i].q[0];
                if constexpr (FMT == 2) q = (q >> (4 * half)) & 0x0f0f0f0fu;
                *(pa_u4 *) (st + key * MM_KST8 + 32 * blk + 16 * half) = q;
                continue;
            }
            mm_dequant<FMT>(R[i], half, lo, hi);
            char * dst = tensor ? st + MM_KT + key * MM_VST : st + key * MM_KST;
            dst += 2 * (32 * blk + 16 * half);
            *(pa_u4 *) dst = lo;
            *(pa_u4 *) (dst + 16) = hi;
        }
    };

    // ---- the first two tiles' loads, then the query rows (B operand: lane (h2, n) holds row n, dims 16kk + 8h2 + t)
    load_tile(R0, t0, true);
    __builtin_amdgcn_sched_barrier(0);
    load_tile(R1, t0 + 1, ntiles > 1);
    __builtin_amdgcn_sched_barrier(0);
    mm_h8 Qf[8];                                                     // !EX: fp16 query operands
    pa_u4 Qi[4];                                                     // EX: int8 query quants per block
    uint32_t dqb[4] = {0u, 0u, 0u, 0u};                              // EX: the scale pairs
    uint32_t dcb[4] = {0u, 0u, 0u, 0u};                              // EX, q4_0: the nibble-offset correction pairs
    if constexpr (EX) mm_prep_qi8<FMT>(a, h, row, rlive, h2, Qi, dqb, dcb);
    else mm_prep_q(a, h, row, rlive, h2, Qf);
    // EX: the B operand of the scale products, the (hi, lo) pair of row n at k = 0, 1 (lanes h2 = 0), zero elsewhere
    uint32_t dqw[4], dcw[4];
    #pragma unroll
    for (int b = 0; b < 4; b++) { dqw[b] = h2 == 0 ? dqb[b] : 0u; dcw[b] = h2 == 0 ? dcb[b] : 0u; }
    // EX, q4_0: the correction MFMA's terms k = 8, 9 (lanes h2 = 1) are 1.0 x the (hi, lo) pair of -mref, so its
    // result starts the scores at -mref; mref is kept at values the pair holds exactly
    const uint32_t onew = h2 == 1 ? 0x3C003C00u : 0u;
    uint32_t mcw = 0u;

    // ---- prologue: tile t0 -> stage 0, tile t0 + 2's loads in flight in R0 (t0 + 1's in R1)
    store_tile(R0, 0);
    load_tile(R0, t0 + PF, ntiles > PF);
    mm_lds_barrier();

    mm_f16 O[4];
    #pragma unroll
    for (int db = 0; db < 4; db++) O[db] = (mm_f16){};
    float mref = -INFINITY, mx = -INFINITY, lsum = 0.0f;
    const float sm = a.qmode == 0 && FMT == 0 ? a.scale * MM_LOG2E : MM_LOG2E;   // score -> base-2 logit (!EX)
    float mc = 0.0f;                                                 // EX: mref once it is finite (0 before), the shift
                                                                     // the block dots start from
    const mm_h2 one2 = {(_Float16) 1.0f, (_Float16) 1.0f};

    const int q4 = lane >> 4, s4 = lane & 15;
    // one tile's matrix work on LDS stage `stage` (nvalid keys)
    auto compute = [&](int stage, int nvalid) {
        const char * Kt = smem + stage * MM_STAGE;
        const char * Vt = Kt + MM_KT;

        // ---- LDS reads: K (A operand of S^T, lane (h2, n): key n, dims 16kk + 8h2 .. +7) first; V^T per dim block
        // and 16-key half by two transposing reads (lane 16q + s reads key row 16mi + (8 for the second read) +
        // 4(q >> 1) + s / 4, dims 32db + 16(q & 1) + 4(s % 4) .. +3), which complete under the softmax
        __builtin_amdgcn_s_waitcnt(0xc07f);                          // lgkmcnt(0): the stores and any scalar load done,
        mm_h8 kf[8];                                                 // so the MFMAs below wait for their own reads only
        if constexpr (!EX) {
            #pragma unroll
            for (int kk = 0; kk < 8; kk++) kf[kk] = *(const mm_h8 *) (Kt + n * MM_KST + 32 * kk + 16 * h2);
            __builtin_amdgcn_sched_barrier(0);
        }
        // ---- S^T = K Q'^T, each MFMA followed by the two transposing V reads of one (dim block, key half), so that at
        // most 15 LDS reads are outstanding (the counter's range) and each MFMA waits for its own K read only
        mm_f16 S = (mm_f16){};
        mm_h8 va[4][2];
        auto v_read = [&](int kk) {
            const int db = kk >> 1, mi = kk & 1;
            const char * vb = Vt + (16 * mi + 4 * (q4 >> 1) + (s4 >> 2)) * MM_VST + 2 * (32 * db + 16 * (q4 & 1) + 4 * (s4 & 3));
            const pa_h4 x0 = __builtin_bit_cast(pa_h4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((MM_LDS mm_tr4 *) vb));
            const pa_h4 x1 = __builtin_bit_cast(pa_h4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((MM_LDS mm_tr4 *) (vb + 8 * MM_VST)));
            va[db][mi] = __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
        };
        if constexpr (EX) {
            // per block: the integer dot on the int8 matrix cores (A: key n's quants, dims 32b + 16h2 .. +15, read raw
            // from the tile; B: the query quants), the scale product, and dot * product summed in fp32
            const pa_u2 dk2 = *(const pa_u2 *) (Kt + MM_KT + MM_VT + 8 * n);   // key n's four fp16 block scales
            const uint32_t hmask = h2 == 0 ? 0xffffffffu : 0u;
            pa_u4 kq[4];
            #pragma unroll
            for (int b = 0; b < 4; b++) kq[b] = *(const pa_u4 *) (Kt + n * MM_KST8 + 32 * b + 16 * h2);
            uint32_t dkw4[4];
            #pragma unroll
            for (int b = 0; b < 4; b++) dkw4[b] = pa_perm(0u, dk2[b >> 1], (b & 1) ? 0x03020302u : 0x01000100u) & hmask;
            if constexpr (FMT == 2) {
                // q4_0: the scores start at -mref plus sum_b dk_b(key) * (-8 * qsum_b * dq_b)(row), one MFMA over the
                // blocks' (hi, lo) pairs (k = 2b, 2b + 1) and -mref (k = 8, 9), so that the unsigned nibble dots need no
                // per-score offset
                S = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                    __builtin_bit_cast(mm_h8, (pa_u4){dkw4[0] | onew, dkw4[1], dkw4[2], dkw4[3]}),
                    __builtin_bit_cast(mm_h8, (pa_u4){dcw[0] | mcw, dcw[1], dcw[2], dcw[3]}), (mm_f16){}, 0, 0, 0);
            }
            #pragma unroll
            for (int b = 0; b < 4; b++) {
                const mm_i16 T = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(mm_i4, kq[b]), __builtin_bit_cast(mm_i4, Qi[b]),
                                                                     (mm_i16){}, 0, 0, 0);
                const uint32_t dkw = dkw4[b];
                const mm_f16 Pb = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(mm_h8, (pa_u4){dkw, 0u, 0u, 0u}),
                                                                         __builtin_bit_cast(mm_h8, (pa_u4){dqw[b], 0u, 0u, 0u}),
                                                                         (mm_f16){}, 0, 0, 0);
                #pragma unroll
                for (int v = 0; v < 16; v++) S[v] = fmaf(Pb[v], (float) T[v], b == 0 && FMT == 1 ? -mc : S[v]);
                __builtin_amdgcn_sched_barrier(0);
            }
            #pragma unroll
            for (int kk = 0; kk < 8; kk++) v_read(kk);               // V^T after the block dots, under the softmax
        } else {
            #pragma unroll
            for (int kk = 0; kk < 8; kk++) {
                S = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[kk], Qf[kk], S, 0, 0, 0);
                v_read(kk);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (nvalid < 32) {                                           // keys 8j + 4h2 + i past the page's end
            #pragma unroll
            for (int v = 0; v < 16; v++)
                if (8 * (v / 4) + 4 * h2 + (v % 4) >= nvalid) S[v] = -INFINITY;
        }
        float tm = S[0];
        #pragma unroll
        for (int v = 1; v < 16; v++) tm = fmaxf(tm, S[v]);
        tm = EX ? mm_max32(tm) + mc : mm_max32(tm) * sm;             // row n's tile max, base 2
        if (__builtin_amdgcn_ballot_w64(tm > mref + MM_PMAX)) {
            // rare: move the reference max of every row that needs it (uniform branch)
            float mn = fmaxf(mref, tm);
            if constexpr (EX && FMT == 2) {                          // a value the (hi, lo) pair of -mn holds exactly
                const _Float16 mh = (_Float16) mn, ml = (_Float16) (mn - (float) mh);
                mn = (float) mh + (float) ml;
                const _Float16 nh = -mh, nl = -ml;
                mcw = h2 == 1 ? (uint32_t) __builtin_bit_cast(uint16_t, nh) | ((uint32_t) __builtin_bit_cast(uint16_t, nl) << 16) : 0u;
            }
            const float alpha = mref == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mref - mn);
            #pragma unroll
            for (int db = 0; db < 4; db++) O[db] *= alpha;
            lsum *= alpha;
            mref = mn;
            if constexpr (EX) {                                      // rebase this tile's scores and the start value
                const float dl = mn - mc;
                #pragma unroll
                for (int v = 0; v < 16; v++) S[v] -= dl;
                mc = mn;
            }
        }
        mx = fmaxf(mx, tm);
        mm_h8 P[2];
        #pragma unroll
        for (int v = 0; v < 16; v++)
            P[v / 8][v % 8] = (_Float16) __builtin_amdgcn_exp2f(EX ? S[v] : fmaf(S[v], sm, -mref));
        #pragma unroll
        for (int v = 0; v < 16; v += 2) {                            // the row sum of the fp16 P the PV MFMAs use
            const mm_h2 pp = {P[v / 8][v % 8], P[v / 8][v % 8 + 1]};
            lsum = __builtin_amdgcn_fdot2(pp, one2, lsum, false);
        }

        // ---- O^T += V^T P^T
        #pragma unroll
        for (int db = 0; db < 4; db++)
            #pragma unroll
            for (int mi = 0; mi < 2; mi++) O[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[db][mi], P[mi], O[db], 0, 0, 0);
    };
    // one tile step; Rn holds tile t + 1's raw bytes
    auto step = [&](uint32_t t, MmRaw<FMT> (&Rn)[UPT]) {
        const int stage = t & 1;
        const uint32_t tau = t0 + t;
        cc.seek(a, tau);                                             // before any LDS operation of this step
        const int nvalid = (int) min(32u, cc.nk - 32 * (tau - cc.tb));
        // the next tile's bytes -> the other stage (last read before the previous barrier; past the chunk's end the
        // stage is written and never read), then tile t + 1 + PF's loads into the registers just freed
        const bool nlive = t + 1 + PF < ntiles;
        if (nlive) cl.seek(a, tau + 1 + PF);
        store_tile(Rn, stage ^ 1);
        load_tile(Rn, tau + 1 + PF, nlive);
        if (wlive) compute(stage, nvalid);
        mm_lds_barrier();                                            // this stage is free; the next one is written
    };
    uint32_t t = 0;                                                  // tile t + 1 is in R((t + 1) % 2)
    for (; t + 2 <= ntiles; t += 2) {
        step(t, R1);
        step(t + 1, R0);
    }
    if (t < ntiles) step(t, R1);

    mm_write_out(a, O, mref, mx, lsum, h, row, rlive, h2, c);
}

// The ggml query rounding over quantized K takes the exact block dots at every size (4-wave verify blocks and 8-wave
// prefill chunks); the reference engines' rounding (PA_QMODE_F16) and f16 K take the fp16-operand QK, the Metal
// engine's own arithmetic (K dequantized to half in threadgroup memory, pa-metal.mm:379-487)
template <int FMT, bool EX>
static hipError_t launch_mma_fmt(int nw, bool skip, const AttnArgs & a, uint32_t grid, hipStream_t st, hipEvent_t ev0,
                                 hipEvent_t ev1) {
    switch (nw) {
        case 4:
            if (skip) hipExtLaunchKernelGGL((mma_kernel<FMT, 4, true, EX>), dim3(grid), dim3(256), 0, st, ev0, ev1, 0, a);
            else hipExtLaunchKernelGGL((mma_kernel<FMT, 4, false, EX>), dim3(grid), dim3(256), 0, st, ev0, ev1, 0, a);
            break;
        case 8:
            if (skip) hipExtLaunchKernelGGL((mma_kernel<FMT, 8, true, EX>), dim3(grid), dim3(512), 0, st, ev0, ev1, 0, a);
            else hipExtLaunchKernelGGL((mma_kernel<FMT, 8, false, EX>), dim3(grid), dim3(512), 0, st, ev0, ev1, 0, a);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_mma(int fmt, int nw, bool skip, const AttnArgs & a, uint32_t grid, hipStream_t st, hipEvent_t ev0,
                      hipEvent_t ev1) {
    const bool ex = a.qmode == 0;                                    // PA_QMODE_GGML over quantized K: exact block dots
    if (fmt == 0) return launch_mma_fmt<0, false>(nw, skip, a, grid, st, ev0, ev1);
    if (fmt == 1) return ex ? launch_mma_fmt<1, true>(nw, skip, a, grid, st, ev0, ev1) : launch_mma_fmt<1, false>(nw, skip, a, grid, st, ev0, ev1);
    if (fmt == 2) return ex ? launch_mma_fmt<2, true>(nw, skip, a, grid, st, ev0, ev1) : launch_mma_fmt<2, false>(nw, skip, a, grid, st, ev0, ev1);
    return hipErrorInvalidValue;
}

}  // namespace pa_hip
