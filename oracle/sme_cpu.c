/* sme_cpu.c - CPU restatement of the reference's C-ABI engine (scripts/sme/sme_attn.c) for the oracle's self-check.
 * TEST INFRASTRUCTURE ONLY: linked into oracle/_ref/pa-tool-cpu (the reference's own pa-tool built from its sources) so
 * that pa-tool's fp64 check (pa-tool.cpp:150-176) and its ATTN_BIG consistency check (pa-tool.cpp:214-243) judge this
 * restatement at the reference shape. The product library exports the same symbols from HIP kernels.
 *
 * Semantics followed (sme_attn.c):
 *   - one KV head: Q fp32 rows (row stride qrs), Qs = f16(q*scale) (sme_attn.c:276-280);
 *   - K/V pointers at key 0 of this head, row stride rs; is_q8 0: f16 values, 1: q8_0 blocks dequantized to f16(d*q)
 *     (deq_q8, sme_attn.c:154-161, an fp16 multiply);
 *   - scores in fp32 from fp16 operands (FMOPA fp16->fp32), online softmax per block of bk keys, P rounded to f16 before
 *     P.V (softmax_blk / sme_pv, sme_attn.c:216-243, 78-105), l from the fp32 p;
 *   - m starts at -1e30, l at 0, O at 0 (sme_attn.c:281-282), so an empty call returns (0, -1e30, 0);
 *   - NR (rows) and HD are the reference's compile-time constants 48/256 (phone-attn.h:78-79); PA_NR / PA_HD override.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "pa_oracle.h"

static int g_nr = 0, g_hd = 0;
static void shape(void) {
    if (g_nr) return;
    const char * a = getenv("PA_NR"), * b = getenv("PA_HD");
    g_nr = a ? atoi(a) : 48;
    g_hd = b ? atoi(b) : 256;
}

static float f16r(float x) { return orc_f16_to_f32(orc_f32_to_f16(x)); }

void * sme_ws_new(void) { shape(); return calloc(1, 64); }
void * sme_pipe_new(int nh) { (void) nh; shape(); return calloc(1, 64); }
int sme2_available(void) { return 1; }

void sme_attn_partial(void * w, const float * Q, int qrs, const uint8_t * K, const uint8_t * V, size_t rs,
                      int is_q8, int nk, float scale, int bk, float * O, float * m, float * l) {
    (void) w;
    shape();
    const int NR = g_nr, HD = g_hd;
    if (bk <= 0) bk = 512;
    float * qs = (float *) malloc(sizeof(float) * (size_t) NR * HD);
    float * kk = (float *) malloc(sizeof(float) * (size_t) bk * HD);
    float * vv = (float *) malloc(sizeof(float) * (size_t) bk * HD);
    float * sc = (float *) malloc(sizeof(float) * (size_t) bk);
    for (int r = 0; r < NR; r++) for (int d = 0; d < HD; d++) qs[r * HD + d] = f16r(Q[(size_t) r * qrs + d] * scale);
    for (int r = 0; r < NR; r++) { m[r] = -1e30f; l[r] = 0.0f; }
    memset(O, 0, sizeof(float) * (size_t) NR * HD);
    for (int j0 = 0; j0 < nk; j0 += bk) {
        const int b = nk - j0 < bk ? nk - j0 : bk;
        for (int j = 0; j < b; j++) {
            const uint8_t * kr = K + (size_t) (j0 + j) * rs, * vr = V + (size_t) (j0 + j) * rs;
            if (is_q8) {
                orc_dequantize(ORC_Q8_0, kr, kk + (size_t) j * HD, HD);
                orc_dequantize(ORC_Q8_0, vr, vv + (size_t) j * HD, HD);
                for (int d = 0; d < HD; d++) { kk[j * HD + d] = f16r(kk[j * HD + d]); vv[j * HD + d] = f16r(vv[j * HD + d]); }
            } else {
                orc_dequantize(ORC_F16, kr, kk + (size_t) j * HD, HD);
                orc_dequantize(ORC_F16, vr, vv + (size_t) j * HD, HD);
            }
        }
        for (int r = 0; r < NR; r++) {
            float mx = -INFINITY;
            for (int j = 0; j < b; j++) {
                float a = 0.0f;
                for (int d = 0; d < HD; d++) a += qs[r * HD + d] * kk[j * HD + d];
                sc[j] = a;
                if (a > mx) mx = a;
            }
            const float mn = fmaxf(m[r], mx), alpha = expf(m[r] - mn);
            float * o = O + (size_t) r * HD;
            for (int d = 0; d < HD; d++) o[d] *= alpha;
            float ls = 0.0f;
            for (int j = 0; j < b; j++) {
                const float p = expf(sc[j] - mn), ph = f16r(p);
                ls += p;
                for (int d = 0; d < HD; d++) o[d] += ph * vv[j * HD + d];
            }
            l[r] = l[r] * alpha + ls;
            m[r] = mn;
        }
    }
    free(qs); free(kk); free(vv); free(sc);
}

/* sme_attn.c:448-463: all nkv heads, Q [nkv][NR][HD], head h at K + h*hb; O [nkv][NR][HD], m, l [nkv][NR] */
void sme_attn_pipe(void ** pp, int nw, int nh, const float * Q, const uint8_t * K, const uint8_t * V, size_t rs, size_t hb,
                   int is_q8, int nkv, int nk, float scale, float * O, float * m, float * l) {
    (void) pp; (void) nw; (void) nh;
    shape();
    for (int h = 0; h < nkv; h++) {
        sme_attn_partial(NULL, Q + (size_t) h * g_nr * g_hd, g_hd, K + (size_t) h * hb, V + (size_t) h * hb, rs, is_q8, nk,
                         scale, 512, O + (size_t) h * g_nr * g_hd, m + (size_t) h * g_nr, l + (size_t) h * g_nr);
    }
}
