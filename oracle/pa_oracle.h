/* pa_oracle.h - CPU oracle for the phone-attn old-KV partial-attention path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links or calls this; only tests/, the smoke check in
 * __graft_entry__.py and bench.py's cpu_baseline leg load liboracle.so, and only as the parity reference (or as the
 * timed CPU baseline), never as the thing measured or shipped.
 *
 * What it restates (reference paths relative to the StayLameBro/backburner checkout):
 *   - row / block formats: q8_0 34-byte blocks (fp16 d + 32 int8), q4_0 18-byte blocks (fp16 d + 16 bytes, byte i = element
 *     i in the low nibble and element i+16 in the high nibble), f16 rows: phone-attn/pa-tool.cpp:41-51,
 *     phone-attn/pa-metal.mm:386-399; row per key with the KV heads side by side: scripts/sme/sme_attn.c:13-14.
 *   - the partial-attention contract O = sum_j e^(s_j-m) v_j, l = sum_j e^(s_j-m), m = max_j s_j, s_j = scale q.k_j:
 *     scripts/sme/sme_attn.c:3-5; empty -> (0, -inf, 0): phone-attn/pa-metal.mm:152, 933.
 *   - the fp64 closed form the reference checks against: phone-attn/pa-tool.cpp:150-176, scripts/sme/sme_attn.c:641-676.
 *   - ggml's CPU flash_attn_ext (the parity target named for this path). ggml lives in the un-vendored llama.cpp fork
 *     (.gitmodules:1-3, StayLameBro/backburner-llama.cpp, gitlink commit not recorded in the checkout); restated from
 *     upstream ggml-cpu's ggml_compute_forward_flash_attn_ext_f16 and the scalar quantize_row_q8_0_ref /
 *     quantize_row_q4_0_ref / ggml_vec_dot_q8_0_q8_0 / ggml_vec_dot_q4_0_q8_0 / dequantize_row_q*_0.
 *   - the LSE merge phone-attn/phone-attn.h:231-239 and the reply normalisation phone-attn/phone-attn.h:651-655.
 *   - greedy acceptance (argmax with lowest-index ties, longest matching draft prefix, bonus token): no code in the
 *     reference tree (the fork's LLAMA_BATCHED_ARGMAX, scripts/serve.sh:8-9, 281, 300-302); stated from its definition.
 *
 * How each function is pinned is listed in tests/test_oracle.py (numpy float16, brute force, closed forms, invariants)
 * and tests/test_ref_patool.py (the reference's own fp64 check in pa-tool.cpp driving orc_sme_* below).
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F16 = 0, ORC_Q8_0 = 1, ORC_Q4_0 = 2 };          /* config_req.is_q8 values, phone-attn.h:15, 88 */
enum { ORC_QMODE_GGML = 0,   /* Q quantized to q8_0 (K's vec_dot type), int block dots, then *scale (ggml CPU)      */
       ORC_QMODE_F16 = 1,    /* Q rounded to f16(q*scale) (phone-attn.h:595-599, sme_attn.c:276-280)               */
       ORC_QMODE_EXACT = 2 };/* fp32 Q as given, no rounding (fp64 closed form only)                                */

typedef struct orc_shape {
    uint32_t nkv;   /* KV heads in a row */
    uint32_t rows;  /* query rows per KV head */
    uint32_t hd;    /* head dim (multiple of 32) */
    uint32_t fmt;   /* ORC_F16 / ORC_Q8_0 / ORC_Q4_0 */
    uint32_t rs;    /* bytes per key row (all heads) */
    uint32_t hb;    /* bytes per head inside a row */
    uint32_t qmode; /* ORC_QMODE_* */
    float scale;    /* softmax scale applied to q.k */
} orc_shape;

/* fp16 <-> fp32, IEEE round-to-nearest-even, subnormals, inf and nan kept */
uint16_t orc_f32_to_f16(float f);
float    orc_f16_to_f32(uint16_t h);
void     orc_f32_to_f16_n(const float * x, uint16_t * y, int64_t n);
void     orc_f16_to_f32_n(const uint16_t * x, float * y, int64_t n);

/* bytes per head for a format and head dim: q8_0 hd/32*34, q4_0 hd/32*18, f16 hd*2 */
uint32_t orc_head_bytes(int fmt, int hd);

/* quantizers, n a multiple of 32 (ggml quantize_row_q8_0_ref / quantize_row_q4_0_ref semantics) */
void orc_quantize_q8_0(const float * x, uint8_t * y, int64_t n);
void orc_quantize_q4_0(const float * x, uint8_t * y, int64_t n);
/* the reference harness's generators (pa-tool.cpp:20-40): id = 1/fp16(d), lrintf + clamp (q8_0); signed max (q4_0) */
void orc_quantize_q8_0_patool(const float * x, uint8_t * y, int64_t n);
void orc_quantize_q4_0_patool(const float * x, uint8_t * y, int64_t n);
/* fmt rows -> fp32, n elements (multiple of 32 for quantized formats) */
void orc_dequantize(int fmt, const uint8_t * x, float * y, int64_t n);
void orc_quantize(int fmt, const float * x, uint8_t * y, int64_t n);

/* seeded N(0,1): splitmix64 counter -> Box-Muller; element i of stream `seed` (independent of how the range is split) */
void orc_normal(uint64_t seed, int64_t i0, int64_t n, float * out);

/* Fill n_keys rows of K or V (row stride rs, nkv heads of hd values in fmt) from stream `seed`: element (key j, head h,
 * dim d) is normal(seed, (j*nkv + h)*hd + d) * amp, times `outlier_mul` on `n_outliers` seeded channels per head
 * (channel picks from stream seed^0x6f75746c), then quantized per 32-block with the ggml semantics above. */
void orc_fill_rows(uint64_t seed, int fmt, int nkv, int hd, uint32_t rs, int64_t j0, int64_t n_keys, float amp,
                   int n_outliers, float outlier_mul, uint8_t * rows);
void orc_outlier_channels(uint64_t seed, int nkv, int hd, int n_outliers, int32_t * ch /* [nkv][n_outliers] */);

/* fp64 closed form over keys [0, nk): O [nkv*rows][hd], m, l [nkv*rows] (unnormalised; empty -> 0, -inf, 0).
 * Q fp32 [nkv][rows][hd] unscaled; K/V rows as above. Two passes per row (max, then sums). */
void orc_attn_exact(const orc_shape * s, const float * Q, const uint8_t * K, const uint8_t * V, int64_t nk,
                    double * O, double * m, double * l, int n_threads);

/* ggml-faithful restatement: per row, Q -> K's vec_dot type, online softmax in key order with expf, fp32 V
 * accumulation; returns (VKQ32, M, S) before ggml's final 1/S. qmode must be ORC_QMODE_GGML. */
void orc_attn_ggml(const orc_shape * s, const float * Q, const uint8_t * K, const uint8_t * V, int64_t nk,
                   float * O, float * m, float * l, int n_threads);

/* The CPU baseline (pa_cpu_simd.c): orc_attn_ggml's arithmetic with ggml's x86 vectorization (AVX-512 VNNI or AVX2
 * integer block dots, vector dequant and accumulator updates), equal to orc_attn_ggml bit for bit. q8_0 / q4_0 K and V,
 * ORC_QMODE_GGML, hd a multiple of 32 up to 512 (anything else runs orc_attn_ggml). force_level: -1 = best available,
 * 2 = AVX-512 VNNI, 1 = AVX2, 0 = scalar. Returns the path taken ("avx512-vnni", "avx2" or "scalar"). */
const char * orc_attn_ggml_simd(const orc_shape * s, const float * Q, const uint8_t * K, const uint8_t * V, int64_t nk,
                                float * O, float * m, float * l, int n_threads, int force_level);
/* the best SIMD path this CPU offers to orc_attn_ggml_simd */
const char * orc_simd_path(void);

/* merge partial (O2, m2, l2) into (O, m, l), rows of hd (phone-attn.h:231-239) */
void orc_merge_partial(float * O, float * m, float * l, const float * O2, const float * m2, const float * l2,
                       int64_t rows, int hd);
/* reply normalisation (phone-attn.h:651-655): Oh = f16(O/l) (0 if l <= 0), lse = m + log(l) (-inf if l <= 0) */
void orc_normalise(const float * O, const float * m, const float * l, int64_t rows, int hd, uint16_t * Oh, float * lse);
/* store_rows' q8_0 -> f16 conversion (phone-attn.h:305-319): rows [n] of stride rs -> f16 [n][nkv][hd] */
void orc_store_rows_f16(const uint8_t * src, int64_t n, int nkv, int hd, uint32_t rs, uint32_t hb, uint16_t * dst);
/* the receiver's co-attention merge of a reply (Oh, lse) with its own partial, normalised (phone-attn.h:21, 231-239,
 * 651-655); lse_out may be NULL */
void orc_coattn_merge(const uint16_t * Oh, const float * lse, const float * Oloc, const float * mloc, const float * lloc,
                      int64_t rows, int hd, float * out, float * lse_out);

/* greedy acceptance over logits [n_rows][vocab] fp32 and a draft of n_rows-1 tokens: argmax[i] (lowest index on ties;
 * the first NaN wins, as numpy.argmax), k = length of the longest prefix with argmax[i] == draft[i], bonus = argmax[k]. */
void orc_accept(const float * logits, int n_rows, int64_t vocab, const int32_t * draft, int32_t * argmax,
                int32_t * k, int32_t * bonus);

/* q8_0 of one Q row the way ggml's CPU path converts it (quantize_row_q8_0 reference semantics) */
void orc_quantize_q_row(const float * q, int hd, uint8_t * out);

#ifdef __cplusplus
}
#endif
