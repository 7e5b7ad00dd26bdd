/* phone_attn_hip.h - C ABI of libpa_hip.so: partial attention over the old, quantized KV cache on MI355X (gfx950).
 *
 * Two groups of entry points:
 *
 *  1. The reference's C ABI, same symbols, argument order and meaning as phone-attn/phone-attn.h:63-71 (the CPU engine
 *     in scripts/sme/sme_attn.c:255-463), so pa::server / pa-tool link against this library unchanged. Buffers are host
 *     memory (or device memory from pa_hip_alloc_page); calls are synchronous. The reference fixes the rows per KV head
 *     and the head dim at compile time (NR = 48, HD = 256: phone-attn.h:78-79); here they default to 48/256 and
 *     pa_hip_set_compat_shape() (or PA_NR / PA_HD in the environment) changes them. These functions return void, as in
 *     the reference; a failure leaves m = -inf, l = 0, O = 0 (the reference GPU engine's failure value,
 *     pa-metal.mm:932-937) and sets pa_hip_last_error().
 *
 *  2. The device-resident engine path: one launch sequence per call over a page table of HBM pages (the role of
 *     pa::engine::begin/end, phone-attn.h:170-174, and of the Metal engine's encode_big, pa-metal.mm:674-714). All
 *     tensors are device pointers, work is enqueued on the caller's stream, nothing is copied to the host.
 *
 * Row format (config_req.rs/hb/is_q8, phone-attn.h:88): key j, KV head h starts at page + j*rs + h*hb; q8_0 = 34-byte
 * blocks (fp16 d, 32 int8), q4_0 = 18-byte blocks (fp16 d, byte i = element i low nibble, element i+16 high nibble),
 * f16 = hd halves. Q is fp32 [nkv][rows][hd], unscaled; O is fp32 [nkv][rows][hd] unnormalised, m and l fp32
 * [nkv][rows] with O = sum_j e^(s_j-m) v_j, l = sum_j e^(s_j-m), m = max_j s_j, s_j = scale*q.k_j
 * (sme_attn.c:3-5); no keys -> (0, -inf, 0).
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- 1. reference C ABI (phone-attn.h:63-71) */

/* sme_attn.c:255 sme_ws_new: one workspace per calling thread (here: a HIP stream and staging buffers). Never freed by
 * the reference's callers; pa_hip_ws_free() releases one. */
void * sme_ws_new(void);

/* sme_attn.c:271-306 sme_attn_partial: ONE KV head. Q fp32 [NR][HD] with row stride qrs floats (unscaled); K, V point at
 * key 0's row of this head (base + h*hb); rs = row stride in bytes; is_q8 0 f16 / 1 q8_0 / 2 q4_0; nk keys (the
 * reference requires a multiple of 64; any nk >= 0 works here); bk is accepted and ignored (the GPU kernel tiles
 * itself). Writes O [NR][HD], m [NR], l [NR]. Rounding follows the reference engines: Q as f16(q*scale), K/V
 * dequantized to fp16, fp32 accumulation. An empty call returns m = -1e30 (sme_attn.c:281). */
void sme_attn_partial(void * w, const float * Q, int qrs, const uint8_t * K, const uint8_t * V, size_t rs,
                      int is_q8, int nk, float scale, int bk, float * O, float * m, float * l);

/* phone-attn.h:67: 1 if the engine can run (a gfx950 device is present and the library initialised on it). The
 * server routes non-GPU pages to the sme_* calls only when this returns 1 (phone-attn.h:588, 593). */
int sme2_available(void);

/* sme_attn.c:419 sme_pipe_new(nh): a pipelined-engine handle; here the same object as sme_ws_new (nh is ignored). */
void * sme_pipe_new(int nh);

/* sme_attn.c:437-463 sme_attn_pipe: ALL nkv heads in one call. pp = nw handles from sme_pipe_new (pp[0]'s stream is
 * used; nw, nh are ignored), Q fp32 [nkv][NR][HD] unscaled, K/V at key 0 of head 0 (head h at +h*hb), rs, hb, is_q8,
 * nkv, nk, scale; O [nkv][NR][HD], m, l [nkv][NR]. */
void sme_attn_pipe(void ** pp, int nw, int nh, const float * Q, const uint8_t * K, const uint8_t * V, size_t rs,
                   size_t hb, int is_q8, int nkv, int nk, float scale, float * O, float * m, float * l);

/* ---------------------------------------------------------------- extensions of the reference ABI */

/* Last error of the calling thread ("" if none). No counterpart in the reference (its C ABI has no error channel). */
const char * pa_hip_last_error(void);

/* Rows per KV head and head dim the sme_* entry points assume (default 48 and 256 = phone-attn.h:78-79). hd must be
 * 128 or 256. Returns 0, or -1 for an unsupported shape. Process-wide; set it before the first call. */
int pa_hip_set_compat_shape(int nr, int hd);

/* Release a handle from sme_ws_new / sme_pipe_new (the reference never frees them). */
void pa_hip_ws_free(void * w);

/* No counterpart in the reference (its engines wait without a limit, pa-metal.mm:928-931): wait until the work enqueued
 * on `stream` (a hipStream_t) has finished, for at most timeout_ms (< 0: no limit). Returns 0 when done, -1 on a stream
 * error or when the limit passed first (pa_hip_last_error() says which). The sme_* calls wait through this with the
 * limit PA_HIP_WAIT_MS (environment, default 30000); a call that runs out of time fails like any other (m = -inf,
 * l = 0, O = 0) and its workspace refuses further calls. */
int pa_hip_stream_wait(void * stream, int timeout_ms);

/* No counterpart in the reference: for a process about to exit (the server's signal handler). New sme_* calls fail from
 * now on; waits up to timeout_ms (< 0: no limit) for the ones running to return. Returns 0 when none is left, -1
 * otherwise. */
int pa_hip_shutdown(int timeout_ms);

/* ---------------------------------------------------------------- 2. device-resident engine path */

enum { PA_FMT_F16 = 0, PA_FMT_Q8_0 = 1, PA_FMT_Q4_0 = 2 };   /* config_req.is_q8 (phone-attn.h:15, 88) */
enum { PA_QMODE_GGML = 0,  /* Q -> q8_0 per 32-block like ggml's CPU flash_attn_ext (K's vec_dot type), s = dot*scale */
       PA_QMODE_F16 = 1 }; /* Q -> f16(q*scale) like the reference engines (phone-attn.h:595-599, sme_attn.c:276-280) */

typedef struct pa_hip_shape {
    uint32_t nkv;     /* KV heads per row (config_req.n_head_kv) */
    uint32_t rows;    /* query rows per KV head: 48 at the reference shape, 8*n_tok at GQA 8 */
    uint32_t hd;      /* head dim: 128 or 256 */
    uint32_t fmt;     /* PA_FMT_* */
    uint32_t rs;      /* bytes per key row, all heads (config_req.rs) */
    uint32_t hb;      /* bytes per head inside a row (config_req.hb) */
    uint32_t qmode;   /* PA_QMODE_* */
    float scale;      /* softmax scale */
} pa_hip_shape;

/* A workspace: split-K partials and the prepared Q, grown on demand with hipMalloc. Calls that share a workspace must
 * be ordered (same stream, or synchronised); use one workspace per concurrent stream. A buffer that must grow is
 * replaced, and the old one kept until pa_hip_ws_destroy, so a graph captured earlier stays valid; growth inside a
 * stream capture is refused (-1): make one eager call of the largest shape before capturing. */
typedef struct pa_hip_ws pa_hip_ws;
pa_hip_ws * pa_hip_ws_new(int device);
void pa_hip_ws_destroy(pa_hip_ws * ws);

/* Split-K geometry of this workspace's calls, for tests and tuning (no counterpart in the reference: the Metal engine
 * fixes its chunking, pa-metal.mm:627-646). decode_groups > 0: tile groups per head pair and launch of the decode
 * kernel (<= 8 rows, head dim 128); mma_workgroups > 0: workgroups per launch of the other kernels; 0 restores the
 * default (one round of resident workgroups: 768 decode workgroups for q8_0, 1024 for q4_0). Returns 0 or -1. */
int pa_hip_ws_set_split(pa_hip_ws * ws, int decode_groups, int mma_workgroups);

/* config_req.gpu_chunk (phone-attn.h:88-89, "keys per GPU threadgroup"; the Metal engine's chunk, pa-metal.mm:842): each
 * workgroup of this workspace's calls takes a split-K chunk of about `keys` keys (rounded to the kernels' 32-key tiles);
 * 0 restores the default geometry. pa_hip_ws_set_split's counts, when set, take precedence. Returns 0 or -1. */
int pa_hip_ws_set_chunk_keys(pa_hip_ws * ws, uint32_t keys);

/* engine::alloc_page / free_page (phone-attn.h:168-169): K and V storage of one page in HBM (device pointers, 256-byte
 * aligned). Returns 0 or -1. */
int pa_hip_alloc_page(size_t bytes, void ** k, void ** v);
void pa_hip_free_page(void * k, void * v);

/* The partial attention of one call: n_pages pages, page i holds nkeys[i] keys of rows rs bytes at k_pages[i] /
 * v_pages[i] (device pointers; the host arrays themselves are read during the call only). Q, O, m, l are device
 * pointers laid out as in the header comment. Enqueued on `stream` (a hipStream_t; NULL = the null stream); returns
 * 0 once enqueued, -1 on a bad argument (nothing enqueued, pa_hip_last_error() says why). */
int pa_hip_attn(pa_hip_ws * ws, const pa_hip_shape * shape, const void * const * k_pages, const void * const * v_pages,
                const uint32_t * nkeys, int n_pages, const float * Q, float * O, float * m, float * l, void * stream);

/* No counterpart in the reference: pa_hip_attn for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops that forbid hipMalloc). The same arguments without a workspace; the call's split-K partials go
 * to a fixed device array of PA_HIP_NOALLOC_SCRATCH bytes that each GPU holds from its first such call until the
 * process ends, and the call allocates nothing. The split adapts so the partials fit (a single launch always does);
 * a call over more than 128 pages whose launches cannot each hold one split of the rows is refused (-1). Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU race (order them on one stream). Returns 0 once
 * enqueued, -1 on a bad argument (nothing enqueued). */
#define PA_HIP_NOALLOC_SCRATCH (64u << 20)
int pa_hip_attn_noalloc(const pa_hip_shape * shape, const void * const * k_pages, const void * const * v_pages,
                        const uint32_t * nkeys, int n_pages, const float * Q, float * O, float * m, float * l, void * stream);

/* Greedy acceptance of a draft block (no code in the reference tree: the fork's LLAMA_BATCHED_ARGMAX, serve.sh:8-9, 281):
 * logits fp32 [n_rows][vocab] and draft int32 [n_rows-1] on the device. out (device int32 [2 + n_rows]) receives
 * out[0] = k, the length of the longest prefix with argmax(logits[i]) == draft[i]; out[1] = the bonus token
 * argmax(logits[k]); out[2+i] = argmax(logits[i]) with the lowest index on ties (the first NaN wins, as numpy.argmax).
 * n_rows <= 64. Returns 0 once enqueued, -1 on a bad argument. */
int pa_hip_accept(pa_hip_ws * ws, const float * logits, int n_rows, int64_t vocab, const int32_t * draft, int32_t * out,
                  void * stream);

/* Measurement hook, no counterpart in the reference: the next pa_hip_attn call on this workspace records ev_start
 * (a hipEvent_t) just before its attention kernel and ev_end just after it, on the call's stream, so a caller can time
 * that kernel alone with hipEventElapsedTime. One call consumes the pair. Returns 0. */
int pa_hip_ws_time_next(pa_hip_ws * ws, void * ev_start, void * ev_end);

/* ---------------------------------------------------------------- 3. the reply side (device epilogues) */
/* The ATTN reply of one call in one step: the partial attention of pa_hip_attn, returned in the reply format of
 * phone-attn.h:651-655 - Oh = f16(O / l) (fp16 bits, [nkv][rows][hd]; 0 where l = 0) and lse = m + log l (fp32
 * [nkv][rows]; -inf where l = 0). When the call is split over several workgroups the split-K merge writes this format
 * itself (no fp32 O round trip); a single-chunk call is normalised by one more kernel. Oh must be 8-byte aligned.
 * Returns 0 once enqueued, -1 on a bad argument. */
int pa_hip_attn_reply(pa_hip_ws * ws, const pa_hip_shape * shape, const void * const * k_pages, const void * const * v_pages,
                      const uint32_t * nkeys, int n_pages, const float * Q, uint16_t * Oh, float * lse, void * stream);
/* pa::merge_partial (phone-attn.h:231-239) on the device: fold the partial (O2, m2, l2) into (O, m, l) in place, `rows`
 * rows of hd (128 or 256) floats, m in natural-log units. A row with l2 <= 0 is left as it is; a row with l <= 0 takes
 * the second partial; otherwise M = max(m, m2), O = O e^(m-M) + O2 e^(m2-M), l = l e^(m-M) + l2 e^(m2-M), m = M (the
 * server's merge of the partials of several engines). O and O2 16-byte aligned. Returns 0 or -1. */
int pa_hip_merge_partial(float * O, float * m, float * l, const float * O2, const float * m2, const float * l2,
                         uint64_t rows, uint32_t hd, void * stream);
/* The reply format (phone-attn.h:651-655) of a partial: Oh = f16(O * (1 / l)) (0 where l <= 0), lse = m + log l (-inf
 * where l <= 0). O 16-byte, Oh 8-byte aligned. Returns 0 or -1. */
int pa_hip_normalise(const float * O, const float * m, const float * l, uint64_t rows, uint32_t hd, uint16_t * Oh,
                     float * lse, void * stream);
/* The receiver's co-attention merge: a reply (Oh, lse) enters the receiver's attention as the partial O_unnorm = Oh,
 * S = 1, M = lse (phone-attn.h:21); it is merged with the receiver's own partial over its recent keys (O_loc, m_loc,
 * l_loc) as pa::merge_partial does, and normalised: out = the attention over both key sets (fp32 [rows][hd]; 0 where
 * neither side has keys), lse_out (optional, may be NULL) = its log-sum-exp. Oh 8-byte, O_loc and out 16-byte aligned.
 * No code in the reference tree (the receiver is the fork's Metal flash attention). Returns 0 or -1. */
int pa_hip_coattn_merge(const uint16_t * Oh, const float * lse, const float * O_loc, const float * m_loc, const float * l_loc,
                        uint64_t rows, uint32_t hd, float * out, float * lse_out, void * stream);
/* ---------------------------------------------------------------- 4. KV ingest into HBM pages */
/* APPEND (phone-attn.h:403-421) into device pages: n received rows of K and of V (rs bytes each, the shape's row
 * format) stored at positions pos0 .. pos0+n-1 of a layer whose page i holds positions [i*page_keys, (i+1)*page_keys)
 * (k_pages / v_pages: host arrays of n_pages device pointers, from pa_hip_alloc_page). store_f16 with fmt q8_0 stores
 * each row as f16 values f16(d*q) instead (store_rows, phone-attn.h:305-319: stored row stride nkv*hd*2, head stride
 * hd*2; other formats are stored as received). K and V may be host memory for the plain copy; the f16 conversion
 * needs device-accessible sources (device memory or pinned host memory) and 4-byte aligned pages. Returns 0 once
 * enqueued, -1 on a bad argument (positions past the last page, a null or misaligned page). */
int pa_hip_append_rows(const pa_hip_shape * shape, void * const * k_pages, void * const * v_pages, int n_pages,
                       uint32_t page_keys, uint32_t pos0, const void * K, const void * V, uint32_t n, int store_f16,
                       void * stream);
/* The sender's side of an APPEND, on the device: K and V fp32 [n][nkv][hd] (device pointers) quantized with the
 * library's ggml-semantics q8_0 / q4_0 quantizer (or converted to f16 for fmt f16) straight into the page rows at
 * positions pos0 .. pos0+n-1 (row format: the shape's rs and hb, both even, multiples of 4 for f16; pages aligned
 * alike; K and V 4-byte aligned). No counterpart in the reference tree (the fork quantizes K/V on the Mac before
 * APPEND). Returns 0 or -1. */
int pa_hip_append_f32(const pa_hip_shape * shape, void * const * k_pages, void * const * v_pages, int n_pages,
                      uint32_t page_keys, uint32_t pos0, const float * K, const float * V, uint32_t n, void * stream);
/* q8_0 / q4_0 quantizer of the library (ggml quantize_row_q8_0_ref / q4_0_ref semantics; the q8_0 one prepares Q in
 * PA_QMODE_GGML): n fp32 values (multiple of 32) at x (4-byte aligned) -> blocks at y (2-byte aligned), both device
 * pointers. Returns 0 or -1. */
int pa_hip_quantize(int fmt, const float * x, void * y, int64_t n, void * stream);
/* ---------------------------------------------------------------- 5. The server engine's row layout */
/* The reference server hands its GPU engine ng groups of query rows (pa::engine::begin, phone-attn.h:174-176): qs =
 * f16(q*scale) [ng][nkv][nr][hd], row i of a head = GQA member i / 8, token i % 8 (nr a multiple of 8). This places
 * them, as fp32, in a pa_hip_attn call's Q [nkv][rows][hd] (use PA_QMODE_F16 with scale 1: the values are already
 * scaled f16): the groups back to back (rows = ng*nr; ntok 0 or 8), or, for one group with 1 <= ntok < 8 real tokens,
 * only the real rows (rows = (nr/8)*ntok, member k's token t at k*ntok + t), as the Metal engine packs them
 * (pa::engine::ntok_hint, phone-attn.h:180; pa-metal.mm:630-634, 661-672). Device pointers; qs 8-byte, q 16-byte
 * aligned; hd a multiple of 4. No counterpart as a function in the reference (its engine packs on the host into shared
 * memory). Returns 0 once enqueued, -1 on a bad argument. */
int pa_hip_pack_q(const uint16_t * qs, uint32_t ng, uint32_t nkv, uint32_t nr, uint32_t hd, uint32_t ntok, float * q,
                  void * stream);
/* The server's keep-warm dispatch between calls (pa::engine::warm, phone-attn.h:179; the Metal engine's 32-thread dispatch,
 * pa-metal.mm:955-968): one 64-thread workgroup that does no work, enqueued on `stream` and not waited for. Returns 0,
 * or -1 if the launch failed. */
int pa_hip_warm(void * stream);
/* The way back: a call's (O, m, l) [nkv][rows] (rows as pa_hip_pack_q made them) to the server's rows Os [ng][nkv*nr][hd],
 * ms, ls [ng][nkv*nr]; the rows of tokens the call did not have get (0, -inf, 0), no keys (pa-metal.mm:501-505). Device
 * pointers, O and Os 16-byte aligned. Returns 0 once enqueued, -1 on a bad argument. */
int pa_hip_unpack_rows(const float * O, const float * m, const float * l, uint32_t ng, uint32_t nkv, uint32_t nr,
                       uint32_t hd, uint32_t ntok, float * Os, float * ms, float * ls, void * stream);

#ifdef __cplusplus
}
#endif
