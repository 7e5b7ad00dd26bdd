/* pa_cpu_simd.c - the CPU baseline: orc_attn_ggml's arithmetic, vectorized the way ggml's CPU backend vectorizes it.
 *
 * TEST AND BENCHMARK INFRASTRUCTURE ONLY (part of liboracle.so): bench.py times it as the CPU path beside the GPU, and
 * tests/test_oracle.py checks it bit for bit against the scalar orc_attn_ggml. Nothing in the product links it.
 *
 * What it restates: ggml-cpu's flash_attn_ext for q8_0 / q4_0 K and V (the parity target of the old-KV path; ggml is
 * in the un-vendored llama.cpp fork, .gitmodules:1-3, and restated in pa_oracle.c): per query row, Q converted to
 * q8_0 (K's vec_dot type), per key s = vec_dot(K_j, Q_q) * scale, online softmax with expf, V dequantized to fp32 and
 * accumulated in fp32 (ggml_vec_scale_f32 / ggml_vec_mad_f32), returning (VKQ32, M, S) before the final 1/S.
 *
 * Vectorized parts, as ggml does them on x86: the integer block dot (AVX-512 VNNI vpdpbusd, or AVX2 vpmaddubsw +
 * vpmaddwd, with the sign trick |k| x sign(q, k)), the V row's int8 -> fp32 dequant, and the scale / multiply-add of
 * the 128-float accumulator. Every fp32 operation rounds as in pa_oracle.c (the block dots are exact integers, the
 * block sums and the accumulator updates keep its operation order, no fused multiply-adds), so the result equals
 * orc_attn_ggml's bit for bit; only the instruction count differs.
 *
 * Threading: OpenMP over (KV head, block of rows), rows of a block sharing each key's decoded V row. The block is
 * smaller than 8 rows when 8 would leave threads idle (ggml itself spreads single rows over the threads).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif
#include <immintrin.h>

#include "pa_oracle.h"

#define SIMD_RB 8        /* at most 8 rows per task */
#define SIMD_HD_MAX 512

static float rd_h(const uint8_t * p) { uint16_t h; memcpy(&h, p, 2); return orc_f16_to_f32(h); }

/* ---------------------------------------------------------------- one K row's quants as 32-byte blocks of int8 */
/* q8_0: the block's 32 quants as they are; q4_0: byte j -> element j (low nibble) and j+16 (high nibble), minus 8 */
static void k_block_bytes(int fmt, const uint8_t * blk, int8_t out[32]) {
    if (fmt == ORC_Q8_0) { memcpy(out, blk + 2, 32); return; }
    for (int j = 0; j < 16; j++) {
        out[j] = (int8_t) ((blk[2 + j] & 0x0f) - 8);
        out[j + 16] = (int8_t) ((blk[2 + j] >> 4) - 8);
    }
}

/* ---------------------------------------------------------------- the per-task kernels */
typedef struct {
    const orc_shape * s;
    const uint8_t * K, * V;
    int64_t nk;
} job_t;

/* the score of one key for nr rows: s_i = sum_b isum_b * (dk_b * dq_b) (q8_0) or (isum_b * dk_b) * dq_b (q4_0), block
 * order, times scale (pa_oracle.c dot_q8_0_q8_0 / dot_q4_0_q8_0) */
static inline float score_from_isums(int fmt, const int32_t * isum, const float * dk, const float * dq, int nb, float scale) {
    float sumf = 0.0f;
    for (int b = 0; b < nb; b++) {
        if (fmt == ORC_Q8_0) sumf += (float) isum[b] * (dk[b] * dq[b]);
        else sumf += (float) isum[b] * dk[b] * dq[b];
    }
    return sumf * scale;
}

/* the online-softmax step and V accumulation of one row (pa_oracle.c orc_attn_ggml, ggml_vec_scale_f32 /
 * ggml_vec_mad_f32) - the vector bodies are passed in so each ISA keeps its own */
#define SOFTMAX_STEP(sv, Mi, Si, vkq, SCALE_FN, MAD_FN)                                                              \
    do {                                                                                                             \
        const float Mold = (Mi);                                                                                     \
        float ms = 1.0f, vs = 1.0f;                                                                                  \
        if ((sv) > (Mi)) { (Mi) = (sv); ms = expf(Mold - (Mi)); SCALE_FN((vkq), ms); }                              \
        else vs = expf((sv) - (Mi));                                                                                 \
        MAD_FN((vkq), vs);                                                                                           \
        (Si) = (Si) * ms + vs;                                                                                       \
    } while (0)

/* ------------------------------------------------ AVX-512 VNNI */
__attribute__((target("avx512f,avx512bw,avx512vl,avx512vnni")))
static void task_avx512(const job_t * J, const float * Q, int h, int r0, int nr, float * O, float * m, float * l) {
    const orc_shape * s = J->s;
    const int hd = (int) s->hd, nb = hd / 32, fmt = (int) s->fmt;
    const int bb = fmt == ORC_Q8_0 ? 34 : 18;
    uint8_t qq[SIMD_RB][SIMD_HD_MAX / 32 * 34];
    float dq[SIMD_RB][SIMD_HD_MAX / 32], M[SIMD_RB], S[SIMD_RB];
    float v32[SIMD_HD_MAX] __attribute__((aligned(64)));
    __m256i qv[SIMD_RB][SIMD_HD_MAX / 32];
    for (int i = 0; i < nr; i++) {
        const size_t row = (size_t) h * s->rows + r0 + i;
        orc_quantize_q8_0(Q + row * hd, qq[i], hd);
        for (int b = 0; b < nb; b++) { dq[i][b] = rd_h(qq[i] + b * 34); qv[i][b] = _mm256_loadu_si256((const __m256i *) (qq[i] + b * 34 + 2)); }
        M[i] = -INFINITY; S[i] = 0.0f;
        memset(O + row * hd, 0, sizeof(float) * (size_t) hd);
    }
    for (int64_t j = 0; j < J->nk; j++) {
        const uint8_t * kr = J->K + (size_t) j * s->rs + (size_t) h * s->hb;
        const uint8_t * vr = J->V + (size_t) j * s->rs + (size_t) h * s->hb;
        /* v_to_float: int8 (or nibble - 8) -> fp32, times the block's fp16 scale */
        for (int b = 0; b < nb; b++) {
            int8_t vb[32];
            k_block_bytes(fmt, vr + b * bb, vb);
            const __m512 d = _mm512_set1_ps(rd_h(vr + b * bb));
            const __m128i lo = _mm_loadu_si128((const __m128i *) vb), hi = _mm_loadu_si128((const __m128i *) (vb + 16));
            _mm512_store_ps(v32 + 32 * b, _mm512_mul_ps(_mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(lo)), d));
            _mm512_store_ps(v32 + 32 * b + 16, _mm512_mul_ps(_mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(hi)), d));
        }
        float dk[SIMD_HD_MAX / 32];
        __m256i kv[SIMD_HD_MAX / 32], ka[SIMD_HD_MAX / 32];
        for (int b = 0; b < nb; b++) {
            int8_t kb[32];
            k_block_bytes(fmt, kr + b * bb, kb);
            dk[b] = rd_h(kr + b * bb);
            kv[b] = _mm256_loadu_si256((const __m256i *) kb);
            ka[b] = _mm256_abs_epi8(kv[b]);                          /* |k| as u8 (quants are within [-127, 127]) */
        }
        for (int i = 0; i < nr; i++) {
            int32_t isum[SIMD_HD_MAX / 32];
            for (int b = 0; b < nb; b += 4) {                        /* four blocks' dot products, then one reduction */
                __m256i d4[4];
                for (int t = 0; t < 4; t++)
                    d4[t] = b + t < nb ? _mm256_dpbusd_epi32(_mm256_setzero_si256(), ka[b + t], _mm256_sign_epi8(qv[i][b + t], kv[b + t]))
                                       : _mm256_setzero_si256();
                const __m256i h01 = _mm256_hadd_epi32(d4[0], d4[1]), h23 = _mm256_hadd_epi32(d4[2], d4[3]);
                const __m256i h = _mm256_hadd_epi32(h01, h23);       /* [b0 b1 b2 b3 | b0 b1 b2 b3] halves */
                const __m128i r = _mm_add_epi32(_mm256_castsi256_si128(h), _mm256_extracti128_si256(h, 1));
                int32_t t4[4];
                _mm_storeu_si128((__m128i *) t4, r);
                for (int t = 0; t < 4 && b + t < nb; t++) isum[b + t] = t4[t];
            }
            const float sv = score_from_isums(fmt, isum, dk, dq[i], nb, s->scale);
            float * vkq = O + ((size_t) h * s->rows + r0 + i) * hd;
#define SCALE512(p, f) do { const __m512 f_ = _mm512_set1_ps(f); for (int d_ = 0; d_ < hd; d_ += 16) _mm512_storeu_ps((p) + d_, _mm512_mul_ps(_mm512_loadu_ps((p) + d_), f_)); } while (0)
#define MAD512(p, f) do { const __m512 f_ = _mm512_set1_ps(f); for (int d_ = 0; d_ < hd; d_ += 16) _mm512_storeu_ps((p) + d_, _mm512_add_ps(_mm512_loadu_ps((p) + d_), _mm512_mul_ps(_mm512_load_ps(v32 + d_), f_))); } while (0)
            SOFTMAX_STEP(sv, M[i], S[i], vkq, SCALE512, MAD512);
#undef SCALE512
#undef MAD512
        }
    }
    for (int i = 0; i < nr; i++) { m[(size_t) h * s->rows + r0 + i] = M[i]; l[(size_t) h * s->rows + r0 + i] = S[i]; }
}

/* ------------------------------------------------ AVX2 */
__attribute__((target("avx2,f16c")))
static void task_avx2(const job_t * J, const float * Q, int h, int r0, int nr, float * O, float * m, float * l) {
    const orc_shape * s = J->s;
    const int hd = (int) s->hd, nb = hd / 32, fmt = (int) s->fmt;
    const int bb = fmt == ORC_Q8_0 ? 34 : 18;
    uint8_t qq[SIMD_RB][SIMD_HD_MAX / 32 * 34];
    float dq[SIMD_RB][SIMD_HD_MAX / 32], M[SIMD_RB], S[SIMD_RB];
    float v32[SIMD_HD_MAX] __attribute__((aligned(32)));
    __m256i qv[SIMD_RB][SIMD_HD_MAX / 32];
    const __m256i ones = _mm256_set1_epi16(1);
    for (int i = 0; i < nr; i++) {
        const size_t row = (size_t) h * s->rows + r0 + i;
        orc_quantize_q8_0(Q + row * hd, qq[i], hd);
        for (int b = 0; b < nb; b++) { dq[i][b] = rd_h(qq[i] + b * 34); qv[i][b] = _mm256_loadu_si256((const __m256i *) (qq[i] + b * 34 + 2)); }
        M[i] = -INFINITY; S[i] = 0.0f;
        memset(O + row * hd, 0, sizeof(float) * (size_t) hd);
    }
    for (int64_t j = 0; j < J->nk; j++) {
        const uint8_t * kr = J->K + (size_t) j * s->rs + (size_t) h * s->hb;
        const uint8_t * vr = J->V + (size_t) j * s->rs + (size_t) h * s->hb;
        for (int b = 0; b < nb; b++) {
            int8_t vb[32];
            k_block_bytes(fmt, vr + b * bb, vb);
            const __m256 d = _mm256_set1_ps(rd_h(vr + b * bb));
            for (int q = 0; q < 4; q++) {
                const __m128i x = _mm_loadl_epi64((const __m128i *) (vb + 8 * q));
                _mm256_store_ps(v32 + 32 * b + 8 * q, _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(x)), d));
            }
        }
        float dk[SIMD_HD_MAX / 32];
        __m256i kv[SIMD_HD_MAX / 32], ka[SIMD_HD_MAX / 32];
        for (int b = 0; b < nb; b++) {
            int8_t kb[32];
            k_block_bytes(fmt, kr + b * bb, kb);
            dk[b] = rd_h(kr + b * bb);
            kv[b] = _mm256_loadu_si256((const __m256i *) kb);
            ka[b] = _mm256_sign_epi8(kv[b], kv[b]);
        }
        for (int i = 0; i < nr; i++) {
            int32_t isum[SIMD_HD_MAX / 32];
            for (int b = 0; b < nb; b += 4) {
                __m256i d4[4];
                for (int t = 0; t < 4; t++)   /* |k| x sign(q, k): 16-bit pair sums stay below 2 * 127 * 127 < 2^15 */
                    d4[t] = b + t < nb ? _mm256_madd_epi16(_mm256_maddubs_epi16(ka[b + t], _mm256_sign_epi8(qv[i][b + t], kv[b + t])), ones)
                                       : _mm256_setzero_si256();
                const __m256i h01 = _mm256_hadd_epi32(d4[0], d4[1]), h23 = _mm256_hadd_epi32(d4[2], d4[3]);
                const __m256i h = _mm256_hadd_epi32(h01, h23);
                const __m128i r = _mm_add_epi32(_mm256_castsi256_si128(h), _mm256_extracti128_si256(h, 1));
                int32_t t4[4];
                _mm_storeu_si128((__m128i *) t4, r);
                for (int t = 0; t < 4 && b + t < nb; t++) isum[b + t] = t4[t];
            }
            const float sv = score_from_isums(fmt, isum, dk, dq[i], nb, s->scale);
            float * vkq = O + ((size_t) h * s->rows + r0 + i) * hd;
#define SCALE256(p, f) do { const __m256 f_ = _mm256_set1_ps(f); for (int d_ = 0; d_ < hd; d_ += 8) _mm256_storeu_ps((p) + d_, _mm256_mul_ps(_mm256_loadu_ps((p) + d_), f_)); } while (0)
#define MAD256(p, f) do { const __m256 f_ = _mm256_set1_ps(f); for (int d_ = 0; d_ < hd; d_ += 8) _mm256_storeu_ps((p) + d_, _mm256_add_ps(_mm256_loadu_ps((p) + d_), _mm256_mul_ps(_mm256_load_ps(v32 + d_), f_))); } while (0)
            SOFTMAX_STEP(sv, M[i], S[i], vkq, SCALE256, MAD256);
#undef SCALE256
#undef MAD256
        }
    }
    for (int i = 0; i < nr; i++) { m[(size_t) h * s->rows + r0 + i] = M[i]; l[(size_t) h * s->rows + r0 + i] = S[i]; }
}

/* ---------------------------------------------------------------- entry point */
static int simd_level(void) {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") && __builtin_cpu_supports("avx512vl") &&
        __builtin_cpu_supports("avx512vnni"))
        return 2;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("f16c")) return 1;
    return 0;
}

const char * orc_simd_path(void) {
    const int lv = simd_level();
    return lv == 2 ? "avx512-vnni" : lv == 1 ? "avx2" : "scalar";
}

const char * orc_attn_ggml_simd(const orc_shape * s, const float * Q, const uint8_t * K, const uint8_t * V, int64_t nk,
                                float * O, float * m, float * l, int n_threads, int force_level) {
    const int lv = force_level >= 0 ? force_level : simd_level();
    if (lv == 0 || s->fmt == ORC_F16 || s->qmode != ORC_QMODE_GGML || s->hd % 32 || s->hd > SIMD_HD_MAX) {
        orc_attn_ggml(s, Q, K, V, nk, O, m, l, n_threads);
        return "scalar";
    }
    int threads = n_threads;
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
    omp_set_num_threads(threads);
#else
    threads = 1;
#endif
    /* rows per task: 8 (a decoded V row serves 8 rows), fewer when 8 would leave threads idle */
    const int rows = (int) s->rows, nkv = (int) s->nkv;
    int rb = SIMD_RB;
    while (rb > 1 && (int64_t) nkv * ((rows + rb - 1) / rb) < 2 * (int64_t) threads) rb /= 2;
    const int nrb = (rows + rb - 1) / rb;
    job_t J = {s, K, V, nk};
    #pragma omp parallel for schedule(dynamic, 1)
    for (int t = 0; t < nkv * nrb; t++) {
        const int h = t / nrb, r0 = (t % nrb) * rb, nr = rows - r0 < rb ? rows - r0 : rb;
        if (lv == 2) task_avx512(&J, Q, h, r0, nr, O, m, l);
        else task_avx2(&J, Q, h, r0, nr, O, m, l);
    }
    return lv == 2 ? "avx512-vnni" : "avx2";
}
