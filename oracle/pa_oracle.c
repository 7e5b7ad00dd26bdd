/* pa_oracle.c - CPU oracle for the phone-attn partial-attention path. TEST INFRASTRUCTURE ONLY (see pa_oracle.h).
 * Built with -ffp-contract=off so every float expression rounds as written. */
#include "pa_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ fp16 */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t mant = x & 0x7fffffu;
    const int32_t exp = (int32_t) ((x >> 23) & 0xffu);
    if (exp == 0xff) return (uint16_t) (sign | 0x7c00u | (mant ? (0x200u | (mant >> 13)) : 0u));
    const int32_t e = exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t) (sign | 0x7c00u);
    if (e <= 0) {                                   /* f16 subnormal (or zero): value / 2^-24 = (1.mant) * 2^(e-14+10) */
        if (e < -10) return (uint16_t) sign;
        mant |= 0x800000u;
        const int shift = 14 - e;
        uint32_t hm = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) hm++;
        return (uint16_t) (sign | hm);
    }
    uint32_t h = sign | ((uint32_t) e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;   /* a carry into the exponent is the correct rounding */
    return (uint16_t) h;
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) x = sign;
        else {                                      /* subnormal: m * 2^-24 */
            float v = (float) m * 5.9604644775390625e-08f;
            memcpy(&x, &v, 4); x |= sign;
        }
    } else if (e == 0x1f) x = sign | 0x7f800000u | (m << 13);
    else x = sign | ((e - 15 + 127) << 23) | (m << 13);
    float f; memcpy(&f, &x, 4);
    return f;
}

void orc_f32_to_f16_n(const float * x, uint16_t * y, int64_t n) { for (int64_t i = 0; i < n; i++) y[i] = orc_f32_to_f16(x[i]); }
void orc_f16_to_f32_n(const uint16_t * x, float * y, int64_t n) { for (int64_t i = 0; i < n; i++) y[i] = orc_f16_to_f32(x[i]); }

uint32_t orc_head_bytes(int fmt, int hd) {
    return fmt == ORC_Q8_0 ? (uint32_t) (hd / 32 * 34) : fmt == ORC_Q4_0 ? (uint32_t) (hd / 32 * 18) : (uint32_t) (hd * 2);
}

static inline float rd_f16(const uint8_t * p) { uint16_t h; memcpy(&h, p, 2); return orc_f16_to_f32(h); }
static inline void wr_f16(uint8_t * p, float f) { const uint16_t h = orc_f32_to_f16(f); memcpy(p, &h, 2); }

/* ------------------------------------------------------------------ quantizers */
/* ggml quantize_row_q8_0_ref: d = amax/127 (fp32), id = 1/d, q = roundf(x*id), d stored as fp16 */
void orc_quantize_q8_0(const float * x, uint8_t * y, int64_t n) {
    for (int64_t b = 0; b < n / 32; b++) {
        const float * xb = x + b * 32;
        uint8_t * o = y + b * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(xb[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        wr_f16(o, d);
        for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t) (int8_t) roundf(xb[j] * id);
    }
}

/* ggml quantize_row_q4_0_ref: signed value of largest magnitude (first one wins), d = max/-8, id = 1/d,
 * q = min(15, (int8_t)(x*id + 8.5)); byte j = q[j] | q[j+16] << 4 */
void orc_quantize_q4_0(const float * x, uint8_t * y, int64_t n) {
    for (int64_t b = 0; b < n / 32; b++) {
        const float * xb = x + b * 32;
        uint8_t * o = y + b * 18;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 32; j++) { const float v = xb[j]; if (amax < fabsf(v)) { amax = fabsf(v); max = v; } }
        const float d = max / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        wr_f16(o, d);
        for (int j = 0; j < 16; j++) {
            const float x0 = xb[j] * id, x1 = xb[16 + j] * id;
            int q0 = (int8_t) (x0 + 8.5f), q1 = (int8_t) (x1 + 8.5f);
            if (q0 > 15) q0 = 15;
            if (q1 > 15) q1 = 15;
            o[2 + j] = (uint8_t) (q0 | (q1 << 4));
        }
    }
}

/* pa-tool.cpp:20-27 make_q8_row: d = am/127, dh = f16(d), id = 1/h2f(dh), q = lrintf(clamp(x*id, -127, 127)) */
void orc_quantize_q8_0_patool(const float * x, uint8_t * y, int64_t n) {
    for (int64_t b = 0; b < n / 32; b++) {
        const float * xb = x + b * 32;
        uint8_t * o = y + b * 34;
        float am = 0.0f;
        for (int j = 0; j < 32; j++) am = fmaxf(am, fabsf(xb[j]));
        const float d = am / 127.0f;
        const uint16_t dh = orc_f32_to_f16(d);
        memcpy(o, &dh, 2);
        const float id = d != 0.0f ? 1.0f / orc_f16_to_f32(dh) : 0.0f;
        for (int j = 0; j < 32; j++) {
            float v = xb[j] * id;
            v = v < -127.0f ? -127.0f : v > 127.0f ? 127.0f : v;
            o[2 + j] = (uint8_t) (int8_t) lrintf(v);
        }
    }
}

/* pa-tool.cpp:29-40 make_q4_row: mx = value of largest |x| (strict >), d = mx/-8, id = 1/h2f(f16(d)),
 * q = clamp((int)(x*id + 8.5), 0, 15) */
void orc_quantize_q4_0_patool(const float * x, uint8_t * y, int64_t n) {
    for (int64_t b = 0; b < n / 32; b++) {
        const float * xb = x + b * 32;
        uint8_t * o = y + b * 18;
        float am = 0.0f, mx = 0.0f;
        for (int j = 0; j < 32; j++) if (fabsf(xb[j]) > am) { am = fabsf(xb[j]); mx = xb[j]; }
        const float d = mx / -8.0f;
        const uint16_t dh = orc_f32_to_f16(d);
        memcpy(o, &dh, 2);
        const float id = d != 0.0f ? 1.0f / orc_f16_to_f32(dh) : 0.0f;
        for (int j = 0; j < 16; j++) {
            int lo = (int) (xb[j] * id + 8.5f), hi = (int) (xb[j + 16] * id + 8.5f);
            lo = lo > 15 ? 15 : lo < 0 ? 0 : lo;
            hi = hi > 15 ? 15 : hi < 0 ? 0 : hi;
            o[2 + j] = (uint8_t) (lo | (hi << 4));
        }
    }
}

/* dequantize_row_q8_0: y = q*d ; dequantize_row_q4_0: y[j] = ((qs[j]&15)-8)*d, y[j+16] = ((qs[j]>>4)-8)*d ; f16 -> f32 */
void orc_dequantize(int fmt, const uint8_t * x, float * y, int64_t n) {
    if (fmt == ORC_Q8_0) {
        for (int64_t b = 0; b < n / 32; b++) {
            const uint8_t * xb = x + b * 34;
            const float d = rd_f16(xb);
            for (int j = 0; j < 32; j++) y[b * 32 + j] = (float) (int8_t) xb[2 + j] * d;
        }
    } else if (fmt == ORC_Q4_0) {
        for (int64_t b = 0; b < n / 32; b++) {
            const uint8_t * xb = x + b * 18;
            const float d = rd_f16(xb);
            for (int j = 0; j < 16; j++) {
                y[b * 32 + j] = (float) ((xb[2 + j] & 0x0f) - 8) * d;
                y[b * 32 + j + 16] = (float) ((xb[2 + j] >> 4) - 8) * d;
            }
        }
    } else {
        for (int64_t i = 0; i < n; i++) y[i] = rd_f16(x + 2 * i);
    }
}

void orc_quantize(int fmt, const float * x, uint8_t * y, int64_t n) {
    if (fmt == ORC_Q8_0) orc_quantize_q8_0(x, y, n);
    else if (fmt == ORC_Q4_0) orc_quantize_q4_0(x, y, n);
    else for (int64_t i = 0; i < n; i++) wr_f16(y + 2 * i, x[i]);
}

void orc_quantize_q_row(const float * q, int hd, uint8_t * out) { orc_quantize_q8_0(q, out, hd); }

/* ------------------------------------------------------------------ synthetic data */
static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
static inline uint64_t stream_word(uint64_t seed, uint64_t p) {   /* splitmix64 stream of mix64(seed), word p */
    return mix64(mix64(seed + 0x9e3779b97f4a7c15ull) + (p + 1) * 0x9e3779b97f4a7c15ull);
}

void orc_normal(uint64_t seed, int64_t i0, int64_t n, float * out) {
    for (int64_t k = 0; k < n; k++) {
        const int64_t i = i0 + k;
        const uint64_t w = stream_word(seed, (uint64_t) (i >> 1));
        const double u1 = (double) ((w >> 40) + 1) * (1.0 / 16777216.0);           /* (0, 1] */
        const double u2 = (double) ((w >> 16) & 0xffffffu) * (1.0 / 16777216.0);   /* [0, 1) */
        const double r = sqrt(-2.0 * log(u1)), t = 6.283185307179586476925 * u2;
        out[k] = (float) ((i & 1) ? r * sin(t) : r * cos(t));
    }
}

void orc_outlier_channels(uint64_t seed, int nkv, int hd, int n_outliers, int32_t * ch) {
    int32_t * perm = (int32_t *) malloc(sizeof(int32_t) * (size_t) hd);
    for (int h = 0; h < nkv; h++) {
        for (int d = 0; d < hd; d++) perm[d] = d;
        for (int i = 0; i < n_outliers && i < hd; i++) {   /* partial Fisher-Yates */
            const uint64_t w = stream_word(seed ^ 0x6f75746c69657273ull, (uint64_t) h * 1024u + (uint64_t) i);
            const int j = i + (int) (w % (uint64_t) (hd - i));
            const int32_t t = perm[i]; perm[i] = perm[j]; perm[j] = t;
            ch[h * n_outliers + i] = perm[i];
        }
    }
    free(perm);
}

void orc_fill_rows(uint64_t seed, int fmt, int nkv, int hd, uint32_t rs, int64_t j0, int64_t n_keys, float amp,
                   int n_outliers, float outlier_mul, uint8_t * rows) {
    const uint32_t hb = orc_head_bytes(fmt, hd);
    int32_t * ch = NULL;
    if (n_outliers > 0) { ch = (int32_t *) malloc(sizeof(int32_t) * (size_t) (nkv * n_outliers)); orc_outlier_channels(seed, nkv, hd, n_outliers, ch); }
    #pragma omp parallel
    {
        float * x = (float *) malloc(sizeof(float) * (size_t) hd);
        #pragma omp for schedule(static)
        for (int64_t jj = 0; jj < n_keys; jj++) {
            const int64_t j = j0 + jj;
            for (int h = 0; h < nkv; h++) {
                orc_normal(seed, (j * nkv + h) * hd, hd, x);
                for (int d = 0; d < hd; d++) x[d] *= amp;
                for (int o = 0; o < n_outliers; o++) x[ch[h * n_outliers + o]] *= outlier_mul;
                orc_quantize(fmt, x, rows + (size_t) jj * rs + (size_t) h * hb, hd);
            }
        }
        free(x);
    }
    free(ch);
}

/* ------------------------------------------------------------------ attention: fp64 closed form */
/* Q row -> the values the dot product sees (double), and the factor applied after the dot */
static void q_effective(const orc_shape * s, const float * q, double * qe, double * post) {
    const int hd = (int) s->hd;
    if (s->qmode == ORC_QMODE_GGML && s->fmt != ORC_F16) {
        uint8_t * qq = (uint8_t *) malloc((size_t) hd / 32 * 34);
        orc_quantize_q8_0(q, qq, hd);
        for (int b = 0; b < hd / 32; b++) {
            const double d = rd_f16(qq + b * 34);
            for (int j = 0; j < 32; j++) qe[b * 32 + j] = d * (double) (int8_t) qq[b * 34 + 2 + j];
        }
        free(qq);
        *post = s->scale;
    } else if (s->qmode == ORC_QMODE_GGML) {      /* f16 K: vec_dot_type is f16, Q converted unscaled */
        for (int d = 0; d < hd; d++) qe[d] = orc_f16_to_f32(orc_f32_to_f16(q[d]));
        *post = s->scale;
    } else if (s->qmode == ORC_QMODE_F16) {       /* f16(q*scale), phone-attn.h:598 */
        for (int d = 0; d < hd; d++) qe[d] = orc_f16_to_f32(orc_f32_to_f16(q[d] * s->scale));
        *post = 1.0;
    } else {
        for (int d = 0; d < hd; d++) qe[d] = q[d];
        *post = s->scale;
    }
}

void orc_attn_exact(const orc_shape * s, const float * Q, const uint8_t * K, const uint8_t * V, int64_t nk,
                    double * O, double * m, double * l, int n_threads) {
    const int hd = (int) s->hd, nrow = (int) (s->nkv * s->rows);
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
#else
    (void) n_threads;
#endif
    #pragma omp parallel
    {
        double * qe = (double *) malloc(sizeof(double) * (size_t) hd);
        double * sc = (double *) malloc(sizeof(double) * (size_t) (nk > 0 ? nk : 1));
        float * kv = (float *) malloc(sizeof(float) * (size_t) hd);
        #pragma omp for schedule(dynamic, 1)
        for (int r = 0; r < nrow; r++) {
            const int h = r / (int) s->rows;
            double post;
            q_effective(s, Q + (size_t) r * hd, qe, &post);
            double mx = -INFINITY;
            for (int64_t j = 0; j < nk; j++) {
                orc_dequantize((int) s->fmt, K + (size_t) j * s->rs + (size_t) h * s->hb, kv, hd);
                double a = 0.0;
                for (int d = 0; d < hd; d++) a += qe[d] * (double) kv[d];
                sc[j] = a * post;
                if (sc[j] > mx) mx = sc[j];
            }
            double L = 0.0, * o = O + (size_t) r * hd;
            for (int d = 0; d < hd; d++) o[d] = 0.0;
            for (int64_t j = 0; j < nk; j++) {
                const double p = exp(sc[j] - mx);
                L += p;
                orc_dequantize((int) s->fmt, V + (size_t) j * s->rs + (size_t) h * s->hb, kv, hd);
                for (int d = 0; d < hd; d++) o[d] += p * (double) kv[d];
            }
            m[r] = nk > 0 ? mx : -INFINITY;
            l[r] = L;
        }
        free(qe); free(sc); free(kv);
    }
}

/* ------------------------------------------------------------------ attention: ggml-faithful */
/* ggml_vec_dot_q8_0_q8_0 (scalar): sumf += sumi*(dx*dy) */
static float dot_q8_0_q8_0(const uint8_t * x, const uint8_t * y, int hd) {
    float sumf = 0.0f;
    for (int b = 0; b < hd / 32; b++) {
        const uint8_t * xb = x + b * 34, * yb = y + b * 34;
        int sumi = 0;
        for (int j = 0; j < 32; j++) sumi += (int) (int8_t) xb[2 + j] * (int) (int8_t) yb[2 + j];
        sumf += (float) sumi * (rd_f16(xb) * rd_f16(yb));
    }
    return sumf;
}
/* ggml_vec_dot_q4_0_q8_0 (scalar): sumi0 over low nibbles with y[j], sumi1 over high nibbles with y[j+16],
 * sumf += sumi*dx*dy (left to right) */
static float dot_q4_0_q8_0(const uint8_t * x, const uint8_t * y, int hd) {
    float sumf = 0.0f;
    for (int b = 0; b < hd / 32; b++) {
        const uint8_t * xb = x + b * 18, * yb = y + b * 34;
        int sumi0 = 0, sumi1 = 0;
        for (int j = 0; j < 16; j++) {
            const int v0 = (xb[2 + j] & 0x0f) - 8, v1 = (xb[2 + j] >> 4) - 8;
            sumi0 += v0 * (int) (int8_t) yb[2 + j];
            sumi1 += v1 * (int) (int8_t) yb[2 + j + 16];
        }
        const int sumi = sumi0 + sumi1;
        sumf += (float) sumi * rd_f16(xb) * rd_f16(yb);
    }
    return sumf;
}
/* ggml_vec_dot_f16 (scalar): double accumulation of fp32 products */
static float dot_f16_f16(const uint8_t * x, const uint16_t * y, int hd) {
    double sumf = 0.0;
    for (int d = 0; d < hd; d++) sumf += (double) (rd_f16(x + 2 * d) * orc_f16_to_f32(y[d]));
    return (float) sumf;
}

#define ORC_RB 8   /* rows of one KV head processed together (key loop outside, so a K/V row is decoded once) */

void orc_attn_ggml(const orc_shape * s, const float * Q, const uint8_t * K, const uint8_t * V, int64_t nk,
                   float * O, float * m, float * l, int n_threads) {
    const int hd = (int) s->hd, rows = (int) s->rows, nkv = (int) s->nkv;
    const int nrb = (rows + ORC_RB - 1) / ORC_RB;
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
#else
    (void) n_threads;
#endif
    #pragma omp parallel
    {
        uint8_t * qq = (uint8_t *) malloc((size_t) ORC_RB * (size_t) hd * 2 + 64);   /* Q_q per row (q8_0 or f16) */
        float * v32 = (float *) malloc(sizeof(float) * (size_t) hd);
        #pragma omp for schedule(dynamic, 1)
        for (int t = 0; t < nkv * nrb; t++) {
            const int h = t / nrb, r0 = (t % nrb) * ORC_RB, nr = rows - r0 < ORC_RB ? rows - r0 : ORC_RB;
            const size_t qb = s->fmt == ORC_F16 ? (size_t) hd * 2 : (size_t) hd / 32 * 34;
            float M[ORC_RB], S[ORC_RB];
            for (int i = 0; i < nr; i++) {
                const size_t row = (size_t) h * rows + r0 + i;
                const float * q = Q + row * hd;
                if (s->fmt == ORC_F16) orc_f32_to_f16_n(q, (uint16_t *) (qq + i * qb), hd);  /* q_to_vec_dot = fp32->fp16 */
                else orc_quantize_q8_0(q, qq + i * qb, hd);                                  /* q_to_vec_dot = q8_0 */
                M[i] = -INFINITY; S[i] = 0.0f;
                memset(O + row * hd, 0, sizeof(float) * (size_t) hd);
            }
            for (int64_t j = 0; j < nk; j++) {
                const uint8_t * kr = K + (size_t) j * s->rs + (size_t) h * s->hb;
                const uint8_t * vr = V + (size_t) j * s->rs + (size_t) h * s->hb;
                orc_dequantize((int) s->fmt, vr, v32, hd);                       /* v_to_float */
                for (int i = 0; i < nr; i++) {
                    float sv = s->fmt == ORC_Q8_0 ? dot_q8_0_q8_0(kr, qq + i * qb, hd)
                             : s->fmt == ORC_Q4_0 ? dot_q4_0_q8_0(kr, qq + i * qb, hd)
                                                   : dot_f16_f16(kr, (const uint16_t *) (qq + i * qb), hd);
                    sv = sv * s->scale;
                    const float Mold = M[i];
                    float ms = 1.0f, vs = 1.0f;
                    float * vkq = O + ((size_t) h * rows + r0 + i) * hd;
                    if (sv > M[i]) {
                        M[i] = sv;
                        ms = expf(Mold - M[i]);
                        for (int d = 0; d < hd; d++) vkq[d] *= ms;                 /* ggml_vec_scale_f32 */
                    } else {
                        vs = expf(sv - M[i]);
                    }
                    for (int d = 0; d < hd; d++) vkq[d] += v32[d] * vs;            /* ggml_vec_mad_f32 */
                    S[i] = S[i] * ms + vs;
                }
            }
            for (int i = 0; i < nr; i++) { m[(size_t) h * rows + r0 + i] = M[i]; l[(size_t) h * rows + r0 + i] = S[i]; }
        }
        free(qq); free(v32);
    }
}

/* ------------------------------------------------------------------ merge / normalise / acceptance */
void orc_merge_partial(float * O, float * m, float * l, const float * O2, const float * m2, const float * l2,
                       int64_t rows, int hd) {
    for (int64_t r = 0; r < rows; r++) {
        if (l2[r] <= 0) continue;
        if (l[r] <= 0) { memcpy(O + r * hd, O2 + r * hd, sizeof(float) * (size_t) hd); m[r] = m2[r]; l[r] = l2[r]; continue; }
        const float M = fmaxf(m[r], m2[r]), a = expf(m[r] - M), b = expf(m2[r] - M);
        for (int d = 0; d < hd; d++) O[r * hd + d] = O[r * hd + d] * a + O2[r * hd + d] * b;
        m[r] = M; l[r] = l[r] * a + l2[r] * b;
    }
}

void orc_normalise(const float * O, const float * m, const float * l, int64_t rows, int hd, uint16_t * Oh, float * lse) {
    for (int64_t r = 0; r < rows; r++) {
        const float inv = l[r] > 0 ? 1.0f / l[r] : 0.0f;
        for (int d = 0; d < hd; d++) Oh[r * hd + d] = orc_f32_to_f16(O[r * hd + d] * inv);
        lse[r] = l[r] > 0 ? m[r] + logf(l[r]) : -INFINITY;
    }
}

/* store_rows with store_f16 (phone-attn.h:305-319): n received q8_0 rows (row stride rs, head stride hb) stored as f16
 * rows [n][nkv][hd], element f16(d * q) */
void orc_store_rows_f16(const uint8_t * src, int64_t n, int nkv, int hd, uint32_t rs, uint32_t hb, uint16_t * dst) {
    for (int64_t j = 0; j < n; j++)
        for (int h = 0; h < nkv; h++)
            for (int b = 0; b < hd / 32; b++) {
                const uint8_t * blk = src + (size_t) j * rs + (size_t) h * hb + (size_t) b * 34;
                const float d = rd_f16(blk);
                for (int i = 0; i < 32; i++)
                    dst[((size_t) j * nkv + h) * hd + b * 32 + i] = orc_f32_to_f16(d * (float) (int8_t) blk[2 + i]);
            }
}

/* The receiver's co-attention slot (phone-attn.h:21): the reply (Oh, lse) enters as the partial O_unnorm = Oh, S = 1,
 * M = lse; it is folded into the receiver's partial by orc_merge_partial (phone-attn.h:231-239) and the result is
 * normalised as O * (1 / l) (phone-attn.h:651-652), lse_out = m + log l. A composition of the two reference formulas;
 * the receiver's own kernel is in the un-vendored fork. */
void orc_coattn_merge(const uint16_t * Oh, const float * lse, const float * Oloc, const float * mloc, const float * lloc,
                      int64_t rows, int hd, float * out, float * lse_out) {
    float * O2 = (float *) malloc(sizeof(float) * (size_t) hd);
    for (int64_t r = 0; r < rows; r++) {
        float m = mloc[r], l = lloc[r];
        const float one = 1.0f;
        float * o = out + r * hd;
        memcpy(o, Oloc + r * hd, sizeof(float) * (size_t) hd);
        for (int d = 0; d < hd; d++) O2[d] = orc_f16_to_f32(Oh[r * hd + d]);
        orc_merge_partial(o, &m, &l, O2, &lse[r], &one, 1, hd);
        const float inv = l > 0 ? 1.0f / l : 0.0f;
        for (int d = 0; d < hd; d++) o[d] = o[d] * inv;
        if (lse_out) lse_out[r] = l > 0 ? m + logf(l) : -INFINITY;
    }
    free(O2);
}

void orc_accept(const float * logits, int n_rows, int64_t vocab, const int32_t * draft, int32_t * argmax,
                int32_t * k, int32_t * bonus) {
    for (int i = 0; i < n_rows; i++) {
        const float * x = logits + (size_t) i * (size_t) vocab;
        int64_t best = 0;
        float bv = x[0];
        if (!isnan(bv)) {
            for (int64_t j = 1; j < vocab; j++) {
                const float v = x[j];
                if (isnan(v)) { best = j; break; }
                if (v > bv) { bv = v; best = j; }
            }
        }
        argmax[i] = (int32_t) best;
    }
    int kk = 0;
    while (kk < n_rows - 1 && argmax[kk] == draft[kk]) kk++;
    *k = kk;
    *bonus = argmax[kk];
}
