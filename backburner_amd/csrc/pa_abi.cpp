// pa_abi.cpp - the C ABI of libpa_hip.so (declared in include/phone_attn_hip.h): the reference's sme_* entry points
// (phone-attn.h:63-71) and the device-resident engine path. Host C++ over the HIP runtime; all compute runs in the HIP
// kernels (pa_decode.hip, pa_mma.hip, pa_attn.hip, pa_reply.hip, pa_ingest.hip, pa_accept.hip). There is no CPU
// fallback: without a gfx950 device every call fails loudly. A workspace belongs to the device it was created on;
// calls that use it expect that device to be current.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/phone_attn_hip.h"
#include "pa_attn.h"

using namespace pa_hip;

namespace {

thread_local std::string g_err;

void set_err(const std::string & e) { g_err = e; }
bool hip_ok(hipError_t e, const char * what) {
    if (e == hipSuccess) return true;
    set_err(std::string(what) + ": " + hipGetErrorString(e));
    return false;
}

// ---------------------------------------------------------------- device check (once per process)
int g_dev_state = -1;   // -1 unknown, 0 unusable, 1 usable
std::string g_dev_why;
std::mutex g_dev_mu;

bool device_usable() {
    std::lock_guard<std::mutex> lk(g_dev_mu);
    if (g_dev_state >= 0) return g_dev_state == 1;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void) hipGetLastError();
        g_dev_state = 0; g_dev_why = "no HIP device";
        return false;
    }
    int dev = 0;
    (void) hipGetDevice(&dev);
    hipDeviceProp_t pr;
    if (hipGetDeviceProperties(&pr, dev) != hipSuccess || std::strncmp(pr.gcnArchName, "gfx950", 6) != 0) {
        g_dev_state = 0; g_dev_why = std::string("device is not gfx950: ") + pr.gcnArchName;
        return false;
    }
    g_dev_state = 1;
    return true;
}

uint32_t head_bytes(int fmt, int hd) {
    return fmt == PA_FMT_Q8_0 ? (uint32_t) (hd / 32 * 34) : fmt == PA_FMT_Q4_0 ? (uint32_t) (hd / 32 * 18) : (uint32_t) (hd * 2);
}

}  // namespace

// ---------------------------------------------------------------- the workspace
struct pa_hip_ws {
    int device = 0;
    float * po = nullptr; size_t po_cap = 0;
    float2 * pml = nullptr; size_t pml_cap = 0;
    unsigned long long * apart = nullptr; size_t apart_cap = 0;
    unsigned int * acount = nullptr;
    // buffers replaced by a larger one: a graph captured earlier may still name them, so they live as long as the
    // workspace (growth at least doubles a buffer, so they hold less than the live ones)
    std::vector<void *> retired;
    // split-K geometry overrides (pa_hip_ws_set_split, pa_hip_ws_set_chunk_keys); 0 = the default geometry
    int dec_groups = 0, mma_workgroups = 0;
    uint32_t chunk_keys = 0;
    // the sme_* compatibility path: its own stream, device staging and a pinned host staging area (host rows are copied
    // into it on the calling thread, so every transfer is pinned <-> device); `broken` after a call whose wait timed
    // out (its transfers may still land in the staging areas, so the workspace is not used again)
    hipStream_t stream = nullptr;
    uint8_t * dk = nullptr; size_t dk_cap = 0;
    uint8_t * dv = nullptr; size_t dv_cap = 0;
    float * dq = nullptr; size_t dq_cap = 0;
    float * dout = nullptr; size_t dout_cap = 0;
    char * hst = nullptr; size_t hst_cap = 0;
    bool broken = false;
    // measurement hook (pa_hip_ws_time_next)
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    // pa_hip_attn_reply: (O, m, l) staging
    float * ro = nullptr; size_t ro_cap = 0;
    float * rml = nullptr; size_t rml_cap = 0;
};

namespace {

// A device buffer of the workspace with room for need_bytes. A larger one replaces it when needed: keep_old retires the
// old one (freed with the workspace: the engine path's buffers, which a captured graph may hold), otherwise it is freed
// once the stream is idle (the synchronous sme_* staging). Growth while `st` is being captured is refused: hipMalloc
// would end the capture, and the graph would hold a buffer the next growth replaces.
template <typename T>
bool ensure(pa_hip_ws * ws, T *& p, size_t & cap, size_t need_bytes, hipStream_t st, bool keep_old, const char * what) {
    if (need_bytes <= cap && p) return true;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) {
        set_err(std::string(what) + ": the workspace must grow (" + std::to_string(need_bytes) +
                " bytes) inside a stream capture; make one eager call of the largest shape before capturing");
        return false;
    }
    (void) hipGetLastError();
    const size_t sz = std::max<size_t>({need_bytes, 2 * cap, 256});
    T * np = nullptr;
    if (!hip_ok(hipMalloc((void **) &np, sz), what)) return false;
    if (p) {
        if (keep_old) ws->retired.push_back((void *) p);
        else { (void) hipStreamSynchronize(st); (void) hipFree(p); }
    }
    p = np;
    cap = sz;
    return true;
}

}  // namespace

extern "C" pa_hip_ws * pa_hip_ws_new(int device) {
    if (!device_usable()) { set_err("pa_hip_ws_new: " + g_dev_why); return nullptr; }
    if (!hip_ok(hipSetDevice(device), "hipSetDevice")) return nullptr;
    pa_hip_ws * w = new pa_hip_ws();
    w->device = device;
    if (!hip_ok(hipMalloc((void **) &w->acount, 256), "hipMalloc counter") ||
        !hip_ok(hipMemset(w->acount, 0, 256), "hipMemset counter")) {   // once, at creation; the kernel keeps it zero
        delete w;
        return nullptr;
    }
    return w;
}

extern "C" void pa_hip_ws_destroy(pa_hip_ws * w) {
    if (!w) return;
    if (w->broken) return;   // a timed-out call may still be using its buffers: they are left to the process
    (void) hipDeviceSynchronize();
    for (void * p : {(void *) w->po, (void *) w->pml, (void *) w->apart, (void *) w->acount, (void *) w->dk,
                     (void *) w->dv, (void *) w->dq, (void *) w->dout, (void *) w->ro, (void *) w->rml})
        (void) hipFree(p);
    for (void * p : w->retired) (void) hipFree(p);
    if (w->hst) (void) hipHostFree(w->hst);
    if (w->stream) (void) hipStreamDestroy(w->stream);
    delete w;
}

extern "C" const char * pa_hip_last_error(void) { return g_err.c_str(); }

extern "C" int pa_hip_ws_time_next(pa_hip_ws * ws, void * ev_start, void * ev_end) {
    if (!ws) { set_err("pa_hip_ws_time_next: null workspace"); return -1; }
    ws->ev0 = (hipEvent_t) ev_start; ws->ev1 = (hipEvent_t) ev_end;
    return 0;
}

extern "C" int pa_hip_ws_set_split(pa_hip_ws * ws, int decode_groups, int mma_workgroups) {
    if (!ws || decode_groups < 0 || mma_workgroups < 0) { set_err("pa_hip_ws_set_split: null workspace or negative count"); return -1; }
    ws->dec_groups = decode_groups;
    ws->mma_workgroups = mma_workgroups;
    return 0;
}

extern "C" int pa_hip_ws_set_chunk_keys(pa_hip_ws * ws, uint32_t keys) {
    if (!ws) { set_err("pa_hip_ws_set_chunk_keys: null workspace"); return -1; }
    ws->chunk_keys = keys;
    return 0;
}

extern "C" int pa_hip_alloc_page(size_t bytes, void ** k, void ** v) {
    if (!k || !v) { set_err("pa_hip_alloc_page: null output"); return -1; }
    *k = *v = nullptr;
    if (!device_usable()) { set_err("pa_hip_alloc_page: " + g_dev_why); return -1; }
    if (!hip_ok(hipMalloc(k, bytes), "hipMalloc page K")) return -1;
    if (!hip_ok(hipMalloc(v, bytes), "hipMalloc page V")) { (void) hipFree(*k); *k = nullptr; return -1; }
    return 0;
}

extern "C" void pa_hip_free_page(void * k, void * v) {
    if (k) (void) hipFree(k);
    if (v) (void) hipFree(v);
}

// ---------------------------------------------------------------- the engine path
namespace {

// decode workgroups per launch (two waves each). q8_0: three per CU, one round (at 8 KV heads x 128k keys 56.4-57.0 us
// per layer against 58.3-58.4 at four per CU; 64k and 256k keys alike; counts between them leave a partial second
// round and are slower). q4_0, twice the work per byte: four per CU (45.4-46.4 against 49.5-50.2 us at three).
constexpr int DEC_TARGET_WG_Q8 = 768, DEC_TARGET_WG_Q4 = 1024;

// One call of the engine path: where its split-K slots go, its geometry overrides, its timing events and, for
// pa_hip_attn_reply, the reply target the merge writes instead of (O, m, l).
struct Call {
    pa_hip_ws * ws = nullptr;         // slots in this workspace's buffers (grown on demand) ...
    char * fixed = nullptr;           // ... or in a fixed device array of `cap` bytes (nothing allocated)
    size_t cap = 0;
    int dec_groups = 0, mma_workgroups = 0;
    uint32_t chunk_keys = 0;          // keys per workgroup's chunk (config_req.gpu_chunk); 0 = the default geometry
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    uint16_t * reply_oh = nullptr;
    float * reply_lse = nullptr;
    bool reply_done = false;
    float * po = nullptr;
    float2 * pml = nullptr;

    // slot rows (one row = hd floats of O and a (max, sum) pair) that a fixed array holds; unlimited for a workspace
    uint64_t max_rows(uint32_t hd) const {
        return fixed ? (cap - 256) / ((uint64_t) hd * sizeof(float) + sizeof(float2)) : ~0ull;
    }
    bool slots(uint64_t rows, uint32_t hd, hipStream_t st) {
        const size_t po_b = std::max<uint64_t>(rows, 1) * hd * sizeof(float);
        const size_t pml_b = std::max<uint64_t>(rows, 1) * sizeof(float2);
        if (fixed) {
            if (rows > max_rows(hd)) {
                set_err("the call's split-K slots (" + std::to_string(po_b + pml_b) + " bytes) exceed the fixed scratch (" +
                        std::to_string(cap) + " bytes)");
                return false;
            }
            po = (float *) fixed;
            pml = (float2 *) (fixed + (po_b + 255) / 256 * 256);
            return true;
        }
        if (!ensure(ws, ws->po, ws->po_cap, po_b, st, true, "hipMalloc partials") ||
            !ensure(ws, ws->pml, ws->pml_cap, pml_b, st, true, "hipMalloc partial stats"))
            return false;
        po = ws->po;
        pml = ws->pml;
        return true;
    }
    // the merge of the call's slots: the reply format when asked for, else (O, m, l)
    bool merge(MergeArgs & ma, int hd, hipStream_t st) {
        if (reply_oh) { ma.Oh = reply_oh; ma.lse = reply_lse; reply_done = true; }
        return hip_ok(launch_merge(hd, ma, st), "merge launch");
    }
};

// The launches of a call: pages in groups of MAXP (their pointers travel in the kernel arguments), calling
// f(first page, pages, 32-key tiles, keys) for each group that holds keys.
template <class F> void for_launches(const uint32_t * nkeys, int n_pages, F f) {
    for (int p0 = 0; p0 < n_pages; p0 += MAXP) {
        const int np = std::min(MAXP, n_pages - p0);
        uint64_t tiles = 0, keys = 0;
        for (int i = 0; i < np; i++) { tiles += (nkeys[p0 + i] + 31) / 32; keys += nkeys[p0 + i]; }
        if (tiles) f(p0, np, tiles, keys);
    }
}

// the page table of one launch: page bases, key prefix and 32-key tile prefix
void page_table(AttnArgs & a, const void * const * k_pages, const void * const * v_pages, const uint32_t * nkeys, int p0, int np) {
    uint32_t acc = 0, tacc = 0;
    for (int i = 0; i < np; i++) {
        a.kp[i] = (const uint8_t *) k_pages[p0 + i];
        a.vp[i] = (const uint8_t *) v_pages[p0 + i];
        a.pstart[i] = acc;
        a.cstart[i] = tacc;
        acc += nkeys[p0 + i];
        tacc += (nkeys[p0 + i] + 31) / 32;
    }
    a.pstart[np] = acc;
    a.cstart[np] = tacc;
    a.n_pages = (uint32_t) np;
    // uniform pages: every page but the last holds the same power of two of whole 32-key tiles
    a.ptl = 32u;
    if (np == 1) a.ptl = 31u;
    else if (nkeys[p0] % 32 == 0 && nkeys[p0] > 0) {
        const uint32_t t = nkeys[p0] / 32;
        bool same = (t & (t - 1)) == 0;
        for (int i = 1; same && i + 1 < np; i++) same = nkeys[p0 + i] == nkeys[p0];
        if (same) a.ptl = (uint32_t) __builtin_ctz(t);
    }
}

// With a fixed slot array: the most chunks per launch that let every launch's slots fit (0 if none would), given the
// call's launch count and slot rows per chunk.
uint64_t chunk_cap(const Call & cx, uint32_t n_launch, uint64_t rows_per_chunk, uint32_t hd) {
    const uint64_t max_chunks = cx.max_rows(hd) / rows_per_chunk;
    return n_launch ? max_chunks / n_launch : max_chunks;
}

// decode calls (<= 8 rows per KV head, q8_0 / q4_0, ggml query rounding, head_dim 128): dec_kernel over (tile group,
// head pair) items - group c of G takes the launch's 32-key tiles c, c + G, ... - about DEC_TARGET_WG_Q8 / _Q4
// workgroups per launch, then the merge kernel
int attn_decode(Call & cx, const pa_hip_shape * s, const void * const * k_pages, const void * const * v_pages,
                const uint32_t * nkeys, int n_pages, const float * Q, float * O, float * m, float * l, hipStream_t st) {
    const uint32_t qr = 8;
    const uint64_t rows_per_slot = (uint64_t) s->nkv * qr;
    // tile groups per head pair: at least two tiles per group unless forced (one-tile groups leave each workgroup's
    // first-load latency and slot write unhidden: 4096 keys 9.7 us at 256 workgroups against 11.8 us at 512)
    auto groups = [&](uint64_t tiles, uint64_t cap) {
        const uint64_t target = s->fmt == PA_FMT_Q4_0 ? DEC_TARGET_WG_Q4 : DEC_TARGET_WG_Q8;
        const uint64_t want = cx.dec_groups > 0 ? (uint64_t) cx.dec_groups
                            : cx.chunk_keys > 0 ? (tiles + std::max<uint64_t>(1, cx.chunk_keys / 32) - 1) / std::max<uint64_t>(1, cx.chunk_keys / 32)
                                                : std::min<uint64_t>(std::max<uint64_t>(1, target / (s->nkv / 2)), (tiles + 1) / 2);
        return (uint32_t) std::max<uint64_t>(1, std::min({tiles, want, cap}));
    };
    uint32_t n_launch = 0;
    uint64_t n_slots = 0, cap = ~0ull;
    for_launches(nkeys, n_pages, [&](int, int, uint64_t tiles, uint64_t) { n_launch++; n_slots += groups(tiles, cap); });
    if (cx.fixed && !(n_launch == 1 && n_slots == 1) && n_slots * rows_per_slot > cx.max_rows(s->hd)) {
        cap = chunk_cap(cx, n_launch, rows_per_slot, s->hd);
        if (cap == 0) { set_err("pa_hip_attn_noalloc: " + std::to_string(n_launch) + " launches need more slots than the scratch holds"); return -1; }
        n_slots = 0;
        for_launches(nkeys, n_pages, [&](int, int, uint64_t tiles, uint64_t) { n_slots += groups(tiles, cap); });
    }
    const bool direct = n_launch == 1 && n_slots == 1;
    if (!direct && !cx.slots(n_slots * rows_per_slot, s->hd, st)) return -1;
    uint32_t li = 0, slot0 = 0;
    bool ok = true;
    for_launches(nkeys, n_pages, [&](int p0, int np, uint64_t tiles, uint64_t) {
        if (!ok) return;
        const uint32_t ng = groups(tiles, cap);
        AttnArgs a;
        std::memset(&a, 0, sizeof a);
        page_table(a, k_pages, v_pages, nkeys, p0, np);
        a.n_chunks = ng; a.chunk = 32;
        a.n_items = ng * (s->nkv / 2);
        a.rs = s->rs; a.hb = s->hb; a.nkv = s->nkv; a.rows = s->rows; a.qr = qr; a.nrb = 1; a.slot0 = slot0;
        a.slots = (uint32_t) n_slots;
        a.qmode = s->qmode; a.fused = direct ? 1u : 0u; a.scale = s->scale;
        a.s_mul = s->scale * 1.4426950408889634f;
        a.q = Q; a.po = cx.po; a.pml = cx.pml; a.O = O; a.m = m; a.l = l;
        const uint32_t grid = (a.n_items + 7) / 8 * 8;
        // the timing events (if any) at the start of the first and the end of the last decode kernel
        ok = hip_ok(launch_decode((int) s->fmt, a, grid, st, li == 0 ? cx.ev0 : nullptr, li + 1 == n_launch ? cx.ev1 : nullptr),
                    "decode launch");
        li++;
        slot0 += ng;
    });
    if (!ok) return -1;
    if (direct) return 0;
    MergeArgs ma;
    ma.po = cx.po; ma.pml = cx.pml; ma.O = O; ma.m = m; ma.l = l;
    ma.n_slots = (uint32_t) n_slots; ma.nkv = s->nkv; ma.qr = qr; ma.rows = s->rows;
    ma.sst = 1; ma.rst = n_slots;                                    // row-major slots: a row's slots contiguous
    return cx.merge(ma, (int) s->hd, st) ? 0 : -1;
}

// the matrix-core kernels: many rows per KV head at head dim 128 (verify, prefill: mma_kernel, row blocks of 32*NW
// rows) and fp16-query calls at head dim 256 (mma256_kernel, row blocks of 64 rows), over chunks of 32-key tiles
int attn_mma(Call & cx, const pa_hip_shape * s, const void * const * k_pages, const void * const * v_pages,
             const uint32_t * nkeys, int n_pages, const float * Q, float * O, float * m, float * l, hipStream_t st) {
    // head dim 128: 32 rows per wave, 8 waves above 128 rows (prefill), 4 otherwise (verify, short verify blocks, f16
    // decode); head dim 256: 16 rows per wave, 4 waves (the reference's 48 rows per KV head fill three)
    const bool h256 = s->hd == 256;
    const uint32_t nw = h256 ? 4u : s->rows > 128 ? 8u : 4u, rpw = h256 ? 16u : 32u;
    const uint32_t nrb = (s->rows + rpw * nw - 1) / (rpw * nw), qr = nrb * rpw * nw;
    // one row block with waves past the last row: those waves only stage (with several row blocks the full ones set
    // the time, and the staging-only branch would slow them)
    const bool skip = nrb == 1 && s->rows <= rpw * (nw - 1);
    const uint32_t units = s->nkv * nrb;
    const uint64_t rows_per_slot = (uint64_t) s->nkv * qr;
    // key chunks: by default one round of resident workgroups (one of 8 waves or two of 4 per CU, 256 CUs); a second,
    // partial round costs more than the extra slots save
    const uint64_t target = cx.mma_workgroups > 0 ? (uint64_t) cx.mma_workgroups : 256u * 8 / nw;
    auto chunking = [&](uint64_t tiles, uint64_t cap, uint32_t & tpc) {
        const uint64_t want = std::max<uint64_t>(1, std::min(target / units, cap));
        tpc = (uint32_t) ((tiles + want - 1) / want);
        if (cx.chunk_keys > 0 && cx.mma_workgroups == 0)             // keys per chunk asked for, within the slot cap
            tpc = (uint32_t) std::max<uint64_t>((tiles + std::min(cap, tiles) - 1) / std::min(cap, tiles),
                                                std::max<uint32_t>(1, cx.chunk_keys / 32));
        return (uint32_t) ((tiles + tpc - 1) / tpc);
    };
    uint32_t n_launch = 0, tpc = 0;
    uint64_t n_slots = 0, cap = ~0ull;
    for_launches(nkeys, n_pages, [&](int, int, uint64_t tiles, uint64_t) { n_launch++; n_slots += chunking(tiles, cap, tpc); });
    if (cx.fixed && !(n_launch == 1 && n_slots == 1) && n_slots * rows_per_slot > cx.max_rows(s->hd)) {
        cap = chunk_cap(cx, n_launch, rows_per_slot, s->hd);
        if (cap == 0) { set_err("pa_hip_attn_noalloc: " + std::to_string(n_launch) + " launches need more slots than the scratch holds"); return -1; }
        n_slots = 0;
        for_launches(nkeys, n_pages, [&](int, int, uint64_t tiles, uint64_t) { n_slots += chunking(tiles, cap, tpc); });
    }
    const bool direct = n_launch == 1 && n_slots == 1;
    if (!direct && !cx.slots(n_slots * rows_per_slot, s->hd, st)) return -1;
    uint32_t li = 0, slot0 = 0;
    bool ok = true;
    for_launches(nkeys, n_pages, [&](int p0, int np, uint64_t tiles, uint64_t) {
        if (!ok) return;
        const uint32_t nch = chunking(tiles, cap, tpc);
        AttnArgs a;
        std::memset(&a, 0, sizeof a);
        page_table(a, k_pages, v_pages, nkeys, p0, np);
        a.n_chunks = nch; a.chunk = tpc;
        a.n_items = nch * units;
        a.rs = s->rs; a.hb = s->hb; a.nkv = s->nkv; a.rows = s->rows; a.qr = qr; a.nrb = nrb; a.slot0 = slot0;
        a.slots = (uint32_t) n_slots;
        a.qmode = s->qmode; a.fused = direct ? 1u : 0u; a.scale = s->scale; a.s_mul = 1.4426950408889634f;
        a.q = Q; a.po = cx.po; a.pml = cx.pml; a.O = O; a.m = m; a.l = l;
        const uint32_t grid = (a.n_items + 7) / 8 * 8;
        hipEvent_t e0 = li == 0 ? cx.ev0 : nullptr, e1 = li + 1 == n_launch ? cx.ev1 : nullptr;
        ok = hip_ok(h256 ? launch_mma256((int) s->fmt, skip, a, grid, st, e0, e1)
                         : launch_mma((int) s->fmt, (int) nw, skip, a, grid, st, e0, e1), "mma launch");
        li++;
        slot0 += nch;
    });
    if (!ok) return -1;
    if (direct) return 0;
    MergeArgs ma;
    ma.po = cx.po; ma.pml = cx.pml; ma.O = O; ma.m = m; ma.l = l;
    ma.n_slots = (uint32_t) n_slots; ma.nkv = s->nkv; ma.qr = qr; ma.rows = s->rows;
    ma.sst = 1; ma.rst = n_slots;
    return cx.merge(ma, (int) s->hd, st) ? 0 : -1;
}

// the argument checks every engine-path attention call shares; false (with the message set) on a bad argument
// (the message strings are built on the error path only: a good call allocates nothing on the host either)
bool attn_args_ok(const char * fn, const pa_hip_shape * s, const void * const * k_pages, const void * const * v_pages,
                  const uint32_t * nkeys, int n_pages, const float * Q, const float * O, const float * m, const float * l) {
    auto bad = [&](const std::string & why) { set_err(std::string(fn) + ": " + why); return false; };
    if (!s) return bad("null shape");
    if (s->hd != 128 && s->hd != 256) return bad("hd must be 128 or 256");
    if (s->fmt > PA_FMT_Q4_0) return bad("fmt must be 0 (f16), 1 (q8_0) or 2 (q4_0)");
    if (s->qmode > PA_QMODE_F16) return bad("qmode must be 0 (ggml) or 1 (f16)");
    if (s->nkv == 0 || s->rows == 0) return bad("nkv and rows must be > 0");
    const uint32_t hbmin = head_bytes((int) s->fmt, (int) s->hd);
    if (s->hb < hbmin || (uint64_t) s->rs < (uint64_t) s->nkv * s->hb)
        return bad("hb " + std::to_string(s->hb) + " / rs " + std::to_string(s->rs) + " too small for nkv " +
                   std::to_string(s->nkv) + " heads of " + std::to_string(hbmin) + " bytes");
    // a kernel's per-tile buffer range spans at most 32 rows of rs bytes in 32 bits
    if (s->rs >= (1u << 26)) return bad("rs must be below 2^26 bytes");
    if (n_pages < 0 || (n_pages > 0 && (!k_pages || !v_pages || !nkeys))) return bad("bad page table");
    if (!Q || !O || !m || !l) return bad("null Q/O/m/l");
    if (((uintptr_t) O & 15) || ((uintptr_t) Q & 3)) return bad("O must be 16-byte and Q 4-byte aligned");
    uint64_t total = 0;
    for (int i = 0; i < n_pages; i++) {
        if (nkeys[i] > 0 && (!k_pages[i] || !v_pages[i])) return bad("null page " + std::to_string(i));
        total += nkeys[i];
    }
    if (total > 0xffffffffull) return bad("more than 2^32 - 1 keys");
    return true;
}

// the kernel path of a checked call
int attn_dispatch(Call & cx, const pa_hip_shape * s, const void * const * k_pages, const void * const * v_pages,
                  const uint32_t * nkeys, int n_pages, const float * Q, float * O, float * m, float * l, hipStream_t st) {
    // decode: <= 8 rows per KV head, quantized K/V with heads packed back to back, an even head count (the last head's
    // 16-byte aligned slice then ends with the row), 16-byte rows
    if (s->qmode == PA_QMODE_GGML && (s->fmt == PA_FMT_Q8_0 || s->fmt == PA_FMT_Q4_0) && s->hd == 128 && s->rows <= 8 &&
        s->hb == head_bytes((int) s->fmt, 128) && s->nkv % 2 == 0 && s->rs % 16 == 0)
        return attn_decode(cx, s, k_pages, v_pages, nkeys, n_pages, Q, O, m, l, st);
    // every other head-dim-128 call (verify, prefill, f16 K/V, odd head counts, padded heads)
    if (s->hd == 128) return attn_mma(cx, s, k_pages, v_pages, nkeys, n_pages, Q, O, m, l, st);
    // head dim 256: matrix cores (fp16 queries, or ggml's q8_0 query rounding with exact block dots over quantized K)
    return attn_mma(cx, s, k_pages, v_pages, nkeys, n_pages, Q, O, m, l, st);
}

// no keys at all: (0, -inf, 0) by the merge kernel over zero slots (nothing else is launched)
int attn_empty(Call & cx, const pa_hip_shape * s, float * O, float * m, float * l, hipStream_t st) {
    if (cx.ev0 && !hip_ok(hipEventRecord(cx.ev0, st), "hipEventRecord")) return -1;
    if (cx.ev1 && !hip_ok(hipEventRecord(cx.ev1, st), "hipEventRecord")) return -1;
    MergeArgs ma;
    ma.po = nullptr; ma.pml = nullptr; ma.O = O; ma.m = m; ma.l = l;
    ma.n_slots = 0; ma.nkv = s->nkv; ma.qr = s->rows; ma.rows = s->rows;
    ma.sst = 0; ma.rst = 0;
    return cx.merge(ma, (int) s->hd, st) ? 0 : -1;
}

int attn_call(Call & cx, const pa_hip_shape * s, const void * const * k_pages, const void * const * v_pages,
              const uint32_t * nkeys, int n_pages, const float * Q, float * O, float * m, float * l, hipStream_t st) {
    uint64_t total = 0;
    for (int i = 0; i < n_pages; i++) total += nkeys[i];
    if (total == 0) return attn_empty(cx, s, O, m, l, st);
    return attn_dispatch(cx, s, k_pages, v_pages, nkeys, n_pages, Q, O, m, l, st);
}

}  // namespace

namespace pa_hip {

void set_error(const std::string & e) { set_err(e); }

int attn_fixed_scratch(char * scratch, size_t cap, const pa_hip_shape * s, const void * const * k_pages,
                       const void * const * v_pages, const uint32_t * nkeys, int n_pages, const float * Q, float * O, float * m,
                       float * l, hipStream_t st) {
    if (!scratch || cap < 4096) { set_err("pa_hip_attn_noalloc: no scratch"); return -1; }
    if (!attn_args_ok("pa_hip_attn_noalloc", s, k_pages, v_pages, nkeys, n_pages, Q, O, m, l)) return -1;
    Call cx;
    cx.fixed = scratch;
    cx.cap = cap;
    return attn_call(cx, s, k_pages, v_pages, nkeys, n_pages, Q, O, m, l, st);
}

}  // namespace pa_hip

extern "C" int pa_hip_attn(pa_hip_ws * ws, const pa_hip_shape * s, const void * const * k_pages, const void * const * v_pages,
                           const uint32_t * nkeys, int n_pages, const float * Q, float * O, float * m, float * l, void * stream) {
    if (!ws) { set_err("pa_hip_attn: null workspace"); return -1; }
    if (!attn_args_ok("pa_hip_attn", s, k_pages, v_pages, nkeys, n_pages, Q, O, m, l)) return -1;
    Call cx;
    cx.ws = ws;
    cx.dec_groups = ws->dec_groups; cx.mma_workgroups = ws->mma_workgroups; cx.chunk_keys = ws->chunk_keys;
    cx.ev0 = ws->ev0; cx.ev1 = ws->ev1;
    ws->ev0 = ws->ev1 = nullptr;
    return attn_call(cx, s, k_pages, v_pages, nkeys, n_pages, Q, O, m, l, (hipStream_t) stream);
}

extern "C" int pa_hip_accept(pa_hip_ws * ws, const float * logits, int n_rows, int64_t vocab, const int32_t * draft, int32_t * out,
                             void * stream) {
    if (!ws || !logits || !out || (n_rows > 1 && !draft)) { set_err("pa_hip_accept: null argument"); return -1; }
    if (n_rows < 1 || n_rows > 64) { set_err("pa_hip_accept: n_rows must be 1..64"); return -1; }
    if (vocab < 1 || vocab > 0x7fffffffLL) { set_err("pa_hip_accept: vocab must be 1..2^31-1"); return -1; }
    if ((vocab & 3) == 0 && ((uintptr_t) logits & 15)) { set_err("pa_hip_accept: logits must be 16-byte aligned"); return -1; }
    const int splits = (int) ((vocab + ACCEPT_SEG - 1) / ACCEPT_SEG);   // ACCEPT_SEG values per workgroup (the kernel's slice)
    const size_t need = (size_t) n_rows * splits * sizeof(unsigned long long);
    if (!ensure(ws, ws->apart, ws->apart_cap, need, (hipStream_t) stream, true, "hipMalloc accept partials")) return -1;
    AcceptArgs a;
    a.logits = logits; a.draft = draft; a.out = out; a.part = ws->apart; a.counter = ws->acount;
    a.vocab = vocab; a.n_rows = n_rows; a.splits = splits;
    return hip_ok(launch_accept(a, (hipStream_t) stream), "accept launch") ? 0 : -1;
}

// ---------------------------------------------------------------- 3. the reply side
extern "C" int pa_hip_attn_reply(pa_hip_ws * ws, const pa_hip_shape * s, const void * const * k_pages,
                                 const void * const * v_pages, const uint32_t * nkeys, int n_pages, const float * Q,
                                 uint16_t * Oh, float * lse, void * stream) {
    if (!ws) { set_err("pa_hip_attn_reply: null workspace"); return -1; }
    if (!Oh || !lse) { set_err("pa_hip_attn_reply: null Oh/lse"); return -1; }
    if ((uintptr_t) Oh & 7) { set_err("pa_hip_attn_reply: Oh must be 8-byte aligned"); return -1; }
    if (!s || (s->hd != 128 && s->hd != 256)) { set_err("pa_hip_attn_reply: hd must be 128 or 256"); return -1; }
    hipStream_t st = (hipStream_t) stream;
    const size_t rows = (size_t) s->nkv * s->rows;
    if (!ensure(ws, ws->ro, ws->ro_cap, std::max<size_t>(rows, 1) * s->hd * sizeof(float), st, true, "hipMalloc reply O") ||
        !ensure(ws, ws->rml, ws->rml_cap, std::max<size_t>(rows, 1) * 2 * sizeof(float), st, true, "hipMalloc reply m, l"))
        return -1;
    float * O = ws->ro, * m = ws->rml, * l = ws->rml + rows;
    if (!attn_args_ok("pa_hip_attn_reply", s, k_pages, v_pages, nkeys, n_pages, Q, O, m, l)) return -1;
    Call cx;
    cx.ws = ws;
    cx.dec_groups = ws->dec_groups; cx.mma_workgroups = ws->mma_workgroups; cx.chunk_keys = ws->chunk_keys;
    cx.ev0 = ws->ev0; cx.ev1 = ws->ev1;
    ws->ev0 = ws->ev1 = nullptr;
    cx.reply_oh = Oh; cx.reply_lse = lse;
    const int rc = attn_call(cx, s, k_pages, v_pages, nkeys, n_pages, Q, O, m, l, st);
    if (rc != 0) return rc;
    if (cx.reply_done) return 0;                                      // the split-K merge wrote the reply
    // a single-chunk call wrote (O, m, l) directly: normalise them
    return hip_ok(launch_normalise((int) s->hd, O, m, l, rows, Oh, lse, st), "normalise launch") ? 0 : -1;
}

namespace {
bool rows_ok(const char * fn, uint64_t rows, uint32_t hd) {
    if (hd != 128 && hd != 256) { set_err(std::string(fn) + ": hd must be 128 or 256"); return false; }
    if (rows > (1ull << 24)) { set_err(std::string(fn) + ": more than 2^24 rows"); return false; }   // 2^22 workgroups
    return true;
}
bool aligned(const void * p, uintptr_t a) { return ((uintptr_t) p & (a - 1)) == 0; }
}  // namespace

extern "C" int pa_hip_merge_partial(float * O, float * m, float * l, const float * O2, const float * m2, const float * l2,
                                    uint64_t rows, uint32_t hd, void * stream) {
    if (!rows_ok("pa_hip_merge_partial", rows, hd)) return -1;
    if (rows > 0 && (!O || !m || !l || !O2 || !m2 || !l2)) { set_err("pa_hip_merge_partial: null argument"); return -1; }
    if (!aligned(O, 16) || !aligned(O2, 16)) { set_err("pa_hip_merge_partial: O, O2 must be 16-byte aligned"); return -1; }
    return hip_ok(launch_merge_partial((int) hd, O, m, l, O2, m2, l2, rows, (hipStream_t) stream), "merge_partial launch") ? 0 : -1;
}

extern "C" int pa_hip_normalise(const float * O, const float * m, const float * l, uint64_t rows, uint32_t hd, uint16_t * Oh,
                                float * lse, void * stream) {
    if (!rows_ok("pa_hip_normalise", rows, hd)) return -1;
    if (rows > 0 && (!O || !m || !l || !Oh || !lse)) { set_err("pa_hip_normalise: null argument"); return -1; }
    if (!aligned(O, 16) || !aligned(Oh, 8)) { set_err("pa_hip_normalise: O must be 16-byte and Oh 8-byte aligned"); return -1; }
    return hip_ok(launch_normalise((int) hd, O, m, l, rows, Oh, lse, (hipStream_t) stream), "normalise launch") ? 0 : -1;
}

extern "C" int pa_hip_coattn_merge(const uint16_t * Oh, const float * lse, const float * O_loc, const float * m_loc,
                                   const float * l_loc, uint64_t rows, uint32_t hd, float * out, float * lse_out, void * stream) {
    if (!rows_ok("pa_hip_coattn_merge", rows, hd)) return -1;
    if (rows > 0 && (!Oh || !lse || !O_loc || !m_loc || !l_loc || !out)) { set_err("pa_hip_coattn_merge: null argument"); return -1; }
    if (!aligned(Oh, 8) || !aligned(O_loc, 16) || !aligned(out, 16)) {
        set_err("pa_hip_coattn_merge: Oh must be 8-byte, O_loc and out 16-byte aligned");
        return -1;
    }
    return hip_ok(launch_coattn((int) hd, Oh, lse, O_loc, m_loc, l_loc, rows, out, lse_out, (hipStream_t) stream),
                  "coattn launch") ? 0 : -1;
}

// ---------------------------------------------------------------- 4. KV ingest into HBM pages
namespace {
// shared checks and the page-segment walk of an APPEND: positions pos0 .. pos0+n-1 over pages of page_keys keys
bool append_ok(const char * fn, const pa_hip_shape * s, void * const * kp, void * const * vp, int n_pages, uint32_t page_keys,
               uint32_t pos0, uint32_t n) {
    const std::string f(fn);
    if (!s) { set_err(f + ": null shape"); return false; }
    if (s->hd != 128 && s->hd != 256) { set_err(f + ": hd must be 128 or 256"); return false; }
    if (s->fmt > PA_FMT_Q4_0 || s->nkv == 0) { set_err(f + ": bad fmt or nkv"); return false; }
    const uint32_t hbmin = head_bytes((int) s->fmt, (int) s->hd);
    if (s->hb < hbmin || (uint64_t) s->rs < (uint64_t) s->nkv * s->hb) { set_err(f + ": hb / rs too small"); return false; }
    if (page_keys == 0) { set_err(f + ": page_keys must be > 0"); return false; }
    if (n == 0) return true;
    if ((uint64_t) pos0 + n > (uint64_t) n_pages * page_keys) { set_err(f + ": positions past the last page"); return false; }
    if (!kp || !vp) { set_err(f + ": null page table"); return false; }
    for (uint64_t pi = pos0 / page_keys; pi <= (pos0 + (uint64_t) n - 1) / page_keys; pi++)
        if (!kp[pi] || !vp[pi]) { set_err(f + ": null page " + std::to_string(pi)); return false; }
    if (2ull * std::min(n, page_keys) * s->nkv * (s->hd / 32) >= (1ull << 31)) { set_err(f + ": segment too large"); return false; }
    return true;
}

// the pages that positions [pos0, pos0 + n) touch are al-byte aligned (the ingest kernels store 16- or 32-bit words)
bool pages_aligned(const char * fn, void * const * kp, void * const * vp, uint32_t page_keys, uint32_t pos0, uint32_t n,
                   uintptr_t al) {
    for (uint64_t pi = pos0 / page_keys; n > 0 && pi <= (pos0 + (uint64_t) n - 1) / page_keys; pi++)
        if (((uintptr_t) kp[pi] | (uintptr_t) vp[pi]) & (al - 1)) {
            set_err(std::string(fn) + ": page " + std::to_string(pi) + " is not " + std::to_string(al) + "-byte aligned");
            return false;
        }
    return true;
}
}  // namespace

extern "C" int pa_hip_append_rows(const pa_hip_shape * s, void * const * k_pages, void * const * v_pages, int n_pages,
                                  uint32_t page_keys, uint32_t pos0, const void * K, const void * V, uint32_t n, int store_f16,
                                  void * stream) {
    const bool f16 = store_f16 && s && s->fmt == PA_FMT_Q8_0;      // store_rows converts q8_0 only (phone-attn.h:305)
    const uint32_t srs = s ? (f16 ? s->nkv * s->hd * 2 : s->rs) : 0;
    if (!append_ok("pa_hip_append_rows", s, k_pages, v_pages, n_pages, page_keys, pos0, n)) return -1;
    if (n > 0 && (!K || !V)) { set_err("pa_hip_append_rows: null K/V"); return -1; }
    if (f16 && !pages_aligned("pa_hip_append_rows", k_pages, v_pages, page_keys, pos0, n, 4)) return -1;
    hipStream_t st = (hipStream_t) stream;
    for (uint32_t done = 0; done < n;) {
        const uint32_t pos = pos0 + done, pi = pos / page_keys, off = pos % page_keys;
        const uint32_t take = std::min(n - done, page_keys - off);
        uint8_t * kd = (uint8_t *) k_pages[pi] + (size_t) off * srs;
        uint8_t * vd = (uint8_t *) v_pages[pi] + (size_t) off * srs;
        const uint8_t * ks = (const uint8_t *) K + (size_t) done * s->rs;
        const uint8_t * vs = (const uint8_t *) V + (size_t) done * s->rs;
        if (!f16) {                                                   // rows as received: one copy per page segment
            if (!hip_ok(hipMemcpyAsync(kd, ks, (size_t) take * s->rs, hipMemcpyDefault, st), "hipMemcpyAsync K") ||
                !hip_ok(hipMemcpyAsync(vd, vs, (size_t) take * s->rs, hipMemcpyDefault, st), "hipMemcpyAsync V"))
                return -1;
        } else {
            AppendArgs a;
            a.kdst = kd; a.vdst = vd; a.ksrc = ks; a.vsrc = vs;
            a.n = take; a.nkv = s->nkv; a.hd = s->hd; a.rs = srs; a.hb = s->hd * 2; a.src_rs = s->rs; a.src_hb = s->hb;
            a.fmt = PA_FMT_F16;
            if (!hip_ok(launch_append(false, a, st), "append f16 launch")) return -1;
        }
        done += take;
    }
    return 0;
}

extern "C" int pa_hip_append_f32(const pa_hip_shape * s, void * const * k_pages, void * const * v_pages, int n_pages,
                                 uint32_t page_keys, uint32_t pos0, const float * K, const float * V, uint32_t n, void * stream) {
    if (!append_ok("pa_hip_append_f32", s, k_pages, v_pages, n_pages, page_keys, pos0, n)) return -1;
    if (n > 0 && (!K || !V)) { set_err("pa_hip_append_f32: null K/V"); return -1; }
    if (((uintptr_t) K & 3) || ((uintptr_t) V & 3)) { set_err("pa_hip_append_f32: K/V must be 4-byte aligned"); return -1; }
    const uint32_t al = s->fmt == PA_FMT_F16 ? 4 : 2;                // the stores are 32-bit (f16) or 16-bit words
    if (s->rs % al || s->hb % al) { set_err("pa_hip_append_f32: rs and hb must be multiples of " + std::to_string(al)); return -1; }
    if (!pages_aligned("pa_hip_append_f32", k_pages, v_pages, page_keys, pos0, n, al)) return -1;
    hipStream_t st = (hipStream_t) stream;
    for (uint32_t done = 0; done < n;) {
        const uint32_t pos = pos0 + done, pi = pos / page_keys, off = pos % page_keys;
        const uint32_t take = std::min(n - done, page_keys - off);
        AppendArgs a;
        a.kdst = (uint8_t *) k_pages[pi] + (size_t) off * s->rs;
        a.vdst = (uint8_t *) v_pages[pi] + (size_t) off * s->rs;
        a.ksrc = K + (size_t) done * s->nkv * s->hd;
        a.vsrc = V + (size_t) done * s->nkv * s->hd;
        a.n = take; a.nkv = s->nkv; a.hd = s->hd; a.rs = s->rs; a.hb = s->hb; a.src_rs = 0; a.src_hb = 0;
        a.fmt = (int) s->fmt;
        if (!hip_ok(launch_append(true, a, st), "append quantize launch")) return -1;
        done += take;
    }
    return 0;
}

extern "C" int pa_hip_quantize(int fmt, const float * x, void * y, int64_t n, void * stream) {
    if (fmt != PA_FMT_Q8_0 && fmt != PA_FMT_Q4_0) { set_err("pa_hip_quantize: fmt must be 1 or 2"); return -1; }
    if (n < 0 || n % 32 || (n > 0 && (!x || !y))) { set_err("pa_hip_quantize: n must be a multiple of 32"); return -1; }
    if (((uintptr_t) x & 3) || ((uintptr_t) y & 1)) { set_err("pa_hip_quantize: x must be 4-byte and y 2-byte aligned"); return -1; }
    return hip_ok(launch_quantize(fmt, x, y, n, (hipStream_t) stream), "quantize launch") ? 0 : -1;
}

// ---------------------------------------------------------------- 1. the reference C ABI
namespace {

std::atomic<int> g_nr{0}, g_hd{0};
int env_int(const char * name, int def) { const char * e = getenv(name); return e ? atoi(e) : def; }
// read once per process: the environment (PA_NR, PA_HD) or the reference's compile-time NR = 48, HD = 256
void compat_shape(int & nr, int & hd) {
    if (g_nr.load() == 0) {
        const int a = env_int("PA_NR", 48), b = env_int("PA_HD", 256);
        int z = 0;
        g_nr.compare_exchange_strong(z, a);
        z = 0;
        g_hd.compare_exchange_strong(z, b);
    }
    nr = g_nr.load(); hd = g_hd.load();
}

// where a caller's buffer lives: device memory (used in place), pinned host memory the runtime already owns
// (hipHostMalloc: copied to the device directly), or pageable host memory (copied into pinned staging first)
enum class Mem { device, pinned, pageable };
Mem mem_kind(const void * p) {
    hipPointerAttribute_t at;
    if (hipPointerGetAttributes(&at, p) != hipSuccess) { (void) hipGetLastError(); return Mem::pageable; }
    return at.type == hipMemoryTypeDevice ? Mem::device : at.type == hipMemoryTypeHost ? Mem::pinned : Mem::pageable;
}

void fail_out(float * O, float * m, float * l, size_t rows, int hd) {
    if (O) std::memset(O, 0, sizeof(float) * rows * (size_t) hd);
    for (size_t r = 0; r < rows; r++) { if (m) m[r] = -INFINITY; if (l) l[r] = 0.0f; }
}

// sme_* calls in flight, and the gate pa_hip_shutdown closes (new calls then fail at once)
std::atomic<int> g_compat_inflight{0};
std::atomic<bool> g_compat_closed{false};
struct InFlight {
    InFlight() { g_compat_inflight.fetch_add(1); }
    ~InFlight() { g_compat_inflight.fetch_sub(1); }
};

// wait limit of the synchronous calls (PA_HIP_WAIT_MS, default 30 s): far above any call's run time, so that a stalled
// device or runtime ends the call with an error instead of blocking its thread for good
int wait_limit_ms() {
    static const int v = [] { const int x = env_int("PA_HIP_WAIT_MS", 30000); return x > 0 ? x : 30000; }();
    return v;
}

// pinned host staging of the workspace with room for `need` bytes (its stream is idle between sme_* calls)
bool ensure_pinned(pa_hip_ws * w, size_t need) {
    if (need <= w->hst_cap && w->hst) return true;
    if (w->hst) { (void) hipHostFree(w->hst); w->hst = nullptr; w->hst_cap = 0; }
    const size_t sz = std::max<size_t>({need, 2 * w->hst_cap, 1u << 16});
    void * p = nullptr;
    if (!hip_ok(hipHostMalloc(&p, sz, hipHostMallocDefault), "hipHostMalloc sme_* staging")) return false;
    w->hst = (char *) p; w->hst_cap = sz;
    return true;
}

size_t al256(size_t b) { return (b + 255) / 256 * 256; }

// one synchronous call of the engine path for `nkv` heads at K/V (host or device), reference rounding (f16 Q*scale).
// Pageable host buffers are never handed to the HIP runtime: K/V spans and Q rows are copied into the workspace's
// pinned staging on the calling thread, only pinned <-> device copies are enqueued, and the results come back through
// the same staging. So concurrent calls from several threads (the server's sme_page, phone-attn.h:509-520) never make
// the runtime pin or stage the callers' pageable pages, and a call's host buffers are not touched by a transfer after
// it returns. K/V spans already in pinned memory (the HIP server engine's pages) are copied to the device directly.
// The wait for the stream is bounded (wait_limit_ms).
bool compat_call(pa_hip_ws * w, const float * Q, int qrs, int qhs, const uint8_t * K, const uint8_t * V, size_t rs, size_t hb,
                 int fmt, int nkv, int nk, float scale, float * O, float * m, float * l) {
    InFlight inflight;
    int NR, HD;
    compat_shape(NR, HD);
    const size_t rows = (size_t) nkv * NR;
    if (g_compat_closed.load()) { set_err("sme_*: the library is shut down (pa_hip_shutdown)"); return false; }
    if (!w) { set_err("sme_*: null workspace"); return false; }
    if (w->broken) { set_err("sme_*: workspace unusable after a call that timed out"); return false; }
    if (fmt < 0 || fmt > 2) { set_err("sme_*: is_q8 must be 0, 1 or 2"); return false; }
    if (nk < 0) { set_err("sme_*: nk < 0"); return false; }
    if (nk == 0) {   // sme_attn.c:281-282: m starts at -1e30, l and O at 0
        std::memset(O, 0, sizeof(float) * rows * HD);
        for (size_t r = 0; r < rows; r++) { m[r] = -1e30f; l[r] = 0.0f; }
        return true;
    }
    if (!w->stream && !hip_ok(hipStreamCreateWithFlags(&w->stream, hipStreamNonBlocking), "hipStreamCreate")) return false;
    hipStream_t st = w->stream;
    const uint32_t hbmin = head_bytes(fmt, HD);
    // K/V: device pointers are used in place; host rows are staged (rows [0, nk) of every head in the span)
    const size_t span = (size_t) (nk - 1) * rs + (size_t) (nkv - 1) * hb + hbmin;
    const Mem k_mem = mem_kind(K), v_mem = mem_kind(V);
    const bool k_stage = k_mem == Mem::pageable, v_stage = v_mem == Mem::pageable;
    const size_t q_b = rows * HD * sizeof(float), o_b = rows * (HD + 2) * sizeof(float);
    // pinned layout: [K span][V span][Q][O, m, l] (the spans only for pageable sources)
    const size_t hk_off = 0, hv_off = k_stage ? al256(span) : 0, hq_off = hv_off + (v_stage ? al256(span) : 0);
    const size_t ho_off = hq_off + al256(q_b);
    if (!ensure_pinned(w, ho_off + o_b)) return false;
    const uint8_t * dK = K, * dV = V;
    if (k_mem != Mem::device) {
        if (!ensure(w, w->dk, w->dk_cap, span, st, false, "hipMalloc K staging")) return false;
        const void * src = K;
        if (k_stage) { std::memcpy(w->hst + hk_off, K, span); src = w->hst + hk_off; }
        if (!hip_ok(hipMemcpyAsync(w->dk, src, span, hipMemcpyHostToDevice, st), "K upload")) return false;
        dK = w->dk;
    }
    if (v_mem != Mem::device) {
        if (!ensure(w, w->dv, w->dv_cap, span, st, false, "hipMalloc V staging")) return false;
        const void * src = V;
        if (v_stage) { std::memcpy(w->hst + hv_off, V, span); src = w->hst + hv_off; }
        if (!hip_ok(hipMemcpyAsync(w->dv, src, span, hipMemcpyHostToDevice, st), "V upload")) return false;
        dV = w->dv;
    }
    if (!ensure(w, w->dq, w->dq_cap, q_b, st, false, "hipMalloc Q staging") ||
        !ensure(w, w->dout, w->dout_cap, o_b, st, false, "hipMalloc O staging"))
        return false;
    float * hq = (float *) (w->hst + hq_off);
    for (int h = 0; h < nkv; h++)
        for (int r = 0; r < NR; r++)
            std::memcpy(hq + ((size_t) h * NR + r) * HD, Q + (size_t) h * qhs + (size_t) r * qrs, HD * sizeof(float));
    if (!hip_ok(hipMemcpyAsync(w->dq, hq, q_b, hipMemcpyHostToDevice, st), "Q upload")) return false;
    pa_hip_shape s;
    s.nkv = (uint32_t) nkv; s.rows = (uint32_t) NR; s.hd = (uint32_t) HD; s.fmt = (uint32_t) fmt;
    s.rs = (uint32_t) rs; s.hb = (uint32_t) hb; s.qmode = PA_QMODE_F16; s.scale = scale;
    if (nkv == 1) { s.hb = hbmin; if (s.rs < s.hb) s.rs = s.hb; }
    const void * kp[1] = {dK}, * vp[1] = {dV};
    const uint32_t nkeys[1] = {(uint32_t) nk};
    float * dO = w->dout, * dm = dO + rows * HD, * dl = dm + rows;
    if (pa_hip_attn(w, &s, kp, vp, nkeys, 1, w->dq, dO, dm, dl, st) != 0) return false;
    float * ho = (float *) (w->hst + ho_off);
    if (!hip_ok(hipMemcpyAsync(ho, dO, o_b, hipMemcpyDeviceToHost, st), "O, m, l download")) return false;
    if (pa_hip_stream_wait(st, wait_limit_ms()) != 0) {
        if (hipStreamQuery(st) == hipErrorNotReady) w->broken = true;
        return false;
    }
    std::memcpy(O, ho, rows * HD * sizeof(float));
    std::memcpy(m, ho + rows * HD, rows * sizeof(float));
    std::memcpy(l, ho + rows * (HD + 1), rows * sizeof(float));
    return true;
}

}  // namespace

extern "C" int pa_hip_set_compat_shape(int nr, int hd) {
    if (nr < 1 || nr > 4096 || (hd != 128 && hd != 256)) { set_err("pa_hip_set_compat_shape: nr 1..4096, hd 128 or 256"); return -1; }
    g_nr.store(nr); g_hd.store(hd);
    return 0;
}

extern "C" void * sme_ws_new(void) {
    int dev = 0;
    if (!device_usable()) { set_err("sme_ws_new: " + g_dev_why); return nullptr; }
    (void) hipGetDevice(&dev);
    return pa_hip_ws_new(dev);
}

extern "C" void * sme_pipe_new(int nh) { (void) nh; return sme_ws_new(); }

extern "C" void pa_hip_ws_free(void * w) { pa_hip_ws_destroy((pa_hip_ws *) w); }

extern "C" int pa_hip_stream_wait(void * stream, int timeout_ms) {
    hipStream_t st = (hipStream_t) stream;
    const auto t0 = std::chrono::steady_clock::now();
    for (unsigned spin = 0;; spin++) {
        const hipError_t e = hipStreamQuery(st);
        if (e == hipSuccess) return 0;
        if (e != hipErrorNotReady) { hip_ok(e, "pa_hip_stream_wait"); return -1; }
        (void) hipGetLastError();   // not-ready is a state, not an error of this thread
        const auto ms = std::chrono::duration_cast<std::chrono::milliseconds>(std::chrono::steady_clock::now() - t0).count();
        if (timeout_ms >= 0 && ms >= timeout_ms) {
            set_err("pa_hip_stream_wait: the stream's work did not finish within " + std::to_string(timeout_ms) + " ms");
            return -1;
        }
        // short calls return within microseconds: spin a little, then poll every 50 us
        if (spin < 1000) std::this_thread::yield();
        else std::this_thread::sleep_for(std::chrono::microseconds(50));
    }
}

extern "C" int pa_hip_shutdown(int timeout_ms) {
    g_compat_closed.store(true);
    const auto t0 = std::chrono::steady_clock::now();
    while (g_compat_inflight.load() > 0) {
        const auto ms = std::chrono::duration_cast<std::chrono::milliseconds>(std::chrono::steady_clock::now() - t0).count();
        if (timeout_ms >= 0 && ms >= timeout_ms) {
            set_err("pa_hip_shutdown: " + std::to_string(g_compat_inflight.load()) + " sme_* calls still running");
            return -1;
        }
        std::this_thread::sleep_for(std::chrono::microseconds(200));
    }
    return 0;
}

extern "C" int sme2_available(void) { return device_usable() ? 1 : 0; }

extern "C" void sme_attn_partial(void * w, const float * Q, int qrs, const uint8_t * K, const uint8_t * V, size_t rs,
                                 int is_q8, int nk, float scale, int bk, float * O, float * m, float * l) {
    (void) bk;
    int NR, HD;
    compat_shape(NR, HD);
    if (!compat_call((pa_hip_ws *) w, Q, qrs, 0, K, V, rs, 0, is_q8, 1, nk, scale, O, m, l)) {
        fprintf(stderr, "sme_attn_partial (libpa_hip): %s\n", g_err.c_str());
        fail_out(O, m, l, (size_t) NR, HD);
    }
}

extern "C" void sme_attn_pipe(void ** pp, int nw, int nh, const float * Q, const uint8_t * K, const uint8_t * V, size_t rs,
                              size_t hb, int is_q8, int nkv, int nk, float scale, float * O, float * m, float * l) {
    (void) nw; (void) nh;
    int NR, HD;
    compat_shape(NR, HD);
    pa_hip_ws * w = pp ? (pa_hip_ws *) pp[0] : nullptr;
    if (!compat_call(w, Q, HD, NR * HD, K, V, rs, hb, is_q8, nkv, nk, scale, O, m, l)) {
        fprintf(stderr, "sme_attn_pipe (libpa_hip): %s\n", g_err.c_str());
        fail_out(O, m, l, (size_t) nkv * NR, HD);
    }
}
