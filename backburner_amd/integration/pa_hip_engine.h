// pa_hip_engine.h - the GPU engine of the reference's phone-attn server on an MI355X: a pa::engine (phone-attn.h:166-183,
// the interface the Metal engine implements in pa-metal.mm:674-953) over libpa_hip.so's pa_hip_attn.
//
// Include phone-attn.h first. Pages (alloc_page): page.k / page.v are pinned host memory, where the unchanged server
// stores the rows APPEND receives (store_rows, phone-attn.h:305-319, 418-419); page.hk / page.hv are their copies in HBM,
// which the kernels read. Each page records how many of its rows the HBM copy holds; a call uploads only the rows past
// that count, so a steady decode moves only the rows appended since the last call over PCIe, never the held ones.
// Rows below the count change only after a TRUNCATE (APPEND writes at the held count, phone-attn.h:407): the server
// reports every TRUNCATE and CONFIG to its page engine (phone-attn.h:344, 395, 437), so this engine registers
// `row_tracker()` there (server::set_page_engine, phone-attn.h:248); the tracker lowers the counts of the pages past the
// new end and never takes keys itself (ready() = 0 pages). Without it every call uploads every row it reads.
//
// One call (begin) on the engine's stream: the new rows; the f16 queries as they are (pa_hip_pack_q places them as fp32:
// for one group with ntok_hint < 8 tokens only the 6 x ntok real rows per KV head, pa-metal.mm:630-634, 661-672);
// pa_hip_attn (PA_QMODE_F16, scale 1: Qs is already f16(q*scale)); pa_hip_unpack_rows into the server's
// [ng][nkv*NR] rows ((0, -inf, 0) for the tokens the call did not have); one copy back. end() waits and copies
// (O, m, l) out; it returns the attention's GPU ms.
// Failure: begin() returns false (the server answers "GPU engine failed to start"); end() returns -1 with
// O = 0, m = -inf, l = 0, the Metal engine's failure value (pa-metal.mm:932-937). Every wait on the engine's stream is
// bounded (pa_hip_stream_wait, PA_HIP_WAIT_MS, default 30 s): a stalled call fails instead of blocking the server.
// close() (the process's exit path) refuses further calls and waits until the one in flight has ended.
#pragma once
#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "phone_attn_hip.h"

namespace pa_hip_server {

struct hip_engine : pa::engine {
    std::string error;

    bool init(int device = 0) {
        if (hipSetDevice(device) != hipSuccess) return fail("hipSetDevice");
        ws_ = pa_hip_ws_new(device);
        if (!ws_) return fail(std::string("pa_hip_ws_new: ") + pa_hip_last_error());
        if (hipStreamCreate(&st_) != hipSuccess || hipEventCreate(&e0_) != hipSuccess || hipEventCreate(&e1_) != hipSuccess)
            return fail("stream / events");
        tracker_.e = this;
        return true;
    }
    ~hip_engine() override {
        if (st_ && !idle(wait_ms())) return;   // work still in flight after the limit: leave its buffers to the process
        disarm();
        if (ws_) pa_hip_ws_destroy(ws_);
        (void) hipFree(dbuf_);
        (void) hipHostFree(hbuf_);
        if (e0_) (void) hipEventDestroy(e0_);
        if (e1_) (void) hipEventDestroy(e1_);
        if (st_) (void) hipStreamDestroy(st_);
    }

    // the server's page engine slot: TRUNCATE / CONFIG notices for the uploaded-row counts
    pa::page_engine * row_tracker() { return &tracker_; }

    bool alloc_page(size_t bytes, pa::page & p) override {
        void * k = nullptr, * v = nullptr, * hk = nullptr, * hv = nullptr;
        if (hipHostMalloc(&k, bytes, hipHostMallocDefault) != hipSuccess) return false;
        if (hipHostMalloc(&v, bytes, hipHostMallocDefault) != hipSuccess) { (void) hipHostFree(k); return false; }
        if (pa_hip_alloc_page(bytes, &hk, &hv) != 0) { (void) hipHostFree(k); (void) hipHostFree(v); return false; }
        p.k = (uint8_t *) k; p.v = (uint8_t *) v; p.hk = hk; p.hv = hv;
        std::lock_guard<std::mutex> lk(mu_);
        held_[hk] = held();
        return true;
    }
    void free_page(pa::page & p) override {
        if (!idle(wait_ms())) { p = pa::page(); return; }            // a copy of this page may be in flight: leak it
        {
            std::lock_guard<std::mutex> lk(gate_mu_);
            disarm();                                                // it may name this page
        }
        {
            std::lock_guard<std::mutex> lk(mu_);
            held_.erase(p.hk);
        }
        (void) hipHostFree(p.k); (void) hipHostFree(p.v);
        pa_hip_free_page(p.hk, p.hv);
        p = pa::page();
    }

    bool begin(const pa::page * pages, const uint32_t * nkeys, int n_pages, const uint16_t * Qs, const pa::config_req & cfg,
               int ng) override {
        {
            std::lock_guard<std::mutex> lk(gate_mu_);
            if (closing_) return fail("the engine is closing");
            in_call_ = true;   // until end(), or until this begin() fails
        }
        if (!start(pages, nkeys, n_pages, Qs, cfg, ng)) { leave(); return false; }
        return true;
    }

    double end(float * O, float * m, float * l) override {
        const double r = finish(O, m, l);
        leave();
        return r;
    }

    // the process's exit path: refuse new calls, wait (up to timeout_ms) until the call in flight has ended and the
    // stream is idle. Returns true when idle.
    bool close(int timeout_ms) {
        std::unique_lock<std::mutex> lk(gate_mu_);
        closing_ = true;
        if (!gate_cv_.wait_for(lk, std::chrono::milliseconds(timeout_ms), [this] { return !in_call_; })) return false;
        lk.unlock();
        return !st_ || idle(timeout_ms);
    }

    double exec_ms() const override { return last_ms_; }
    std::string describe() override {
        return "hip MI355X (libpa_hip) rows_uploaded=" + std::to_string(rows_up_) + (tracked_ ? " tracked=1" : " tracked=0") +
               " call_rows_per_kv_head=" + std::to_string(last_rows_) + " armed=" + std::to_string(n_armed_) +
               " armed_hits=" + std::to_string(n_armed_hits_) + " warms=" + std::to_string(n_warm_);
    }
    uint64_t rows_uploaded() const { return rows_up_; }   // K/V rows copied to HBM since init
    uint64_t armed_hits() const { return n_armed_hits_; }  // calls that ran as an armed graph

    // between calls (the server's hot spin, phone-attn.h:356-370): one small dispatch, not waited for, so the device
    // keeps its clocks up; skipped while a call is in flight (as the Metal engine skips it, pa-metal.mm:955-968)
    void warm() override {
        std::lock_guard<std::mutex> lk(gate_mu_);
        if (closing_ || in_call_) return;
        if (pa_hip_warm(st_) == 0) n_warm_++;
    }

    // after a one-group call the server names the likely next call (the next layer, same split and tokens,
    // phone-attn.h:687-697): its whole launch sequence (query copy, packing, attention, unpacking, reply copy) is
    // captured now as a HIP graph, off the critical path, so that the call itself is one memcpy of Q into pinned memory
    // and one graph launch (the Metal engine's pre-encoded command buffer, pa-metal.mm:716-765). A call that does not
    // match it (other pages, key counts, tokens or row format) runs the ordinary launches. Off unless PA_GPU_ARM=1, as
    // in the Metal engine: at 131,072 keys, back-to-back decode calls over loopback measured 0.479 ms per round trip
    // armed against 0.446 ms not (the capture and instantiation run on the server thread after the reply, when a fast
    // client's next call is already waiting).
    void arm(const pa::page * pages, const uint32_t * nkeys, int n_pages, const pa::config_req & cfg, int ntok) override {
        static const bool on = getenv("PA_GPU_ARM") && atoi(getenv("PA_GPU_ARM")) != 0;
        std::lock_guard<std::mutex> lk(gate_mu_);
        disarm();
        if (!on || closing_ || in_call_ || n_pages <= 0) return;
        const call_geom g = geom_of(cfg, 1, ntok);
        if (!ensure(g.dev_bytes(), g.host_bytes())) return;
        (void) pa_hip_ws_set_chunk_keys(ws_, cfg.gpu_chunk);
        if (hipStreamBeginCapture(st_, hipStreamCaptureModeThreadLocal) != hipSuccess) { (void) hipGetLastError(); return; }
        const bool ok = enqueue(pages, nkeys, n_pages, cfg, g, false);
        hipGraph_t graph = nullptr;
        const bool ended = hipStreamEndCapture(st_, &graph) == hipSuccess;
        if (ok && ended && graph && hipGraphInstantiate(&armed_.exec, graph, nullptr, nullptr, 0) == hipSuccess) {
            armed_.hk.resize(n_pages); armed_.nkeys.assign(nkeys, nkeys + n_pages);
            for (int i = 0; i < n_pages; i++) armed_.hk[i] = pages[i].hk;
            armed_.rs = cfg.rs; armed_.hb = cfg.hb; armed_.is_q8 = cfg.is_q8; armed_.nkv = cfg.n_head_kv;
            armed_.chunk = cfg.gpu_chunk; armed_.nt = g.nt;
            n_armed_++;
        } else {
            armed_.exec = nullptr;
            (void) hipGetLastError();
        }
        if (graph) (void) hipGraphDestroy(graph);
    }

private:
    // one call's rows and buffer layout: device qs (f16, server layout) | Q (fp32, call layout) | O, m, l (call) |
    // O, m, l (server); host (pinned): qs | O, m, l (server)
    struct call_geom {
        uint32_t nkv = 0, ng = 1, nt = 0, rows = 0;
        size_t srows = 0, crows = 0, qs_b = 0, q_b = 0, oc_b = 0, os_b = 0;
        size_t dev_bytes() const { return qs_b + q_b + oc_b + os_b; }
        size_t host_bytes() const { return qs_b + os_b; }
    };
    static call_geom geom_of(const pa::config_req & cfg, int ng, int ntok) {
        call_geom g;
        g.nkv = (uint32_t) cfg.n_head_kv; g.ng = (uint32_t) ng;
        g.nt = (ng == 1 && ntok >= 1 && ntok < 8) ? (uint32_t) ntok : 0;
        g.rows = g.nt ? (pa::NR / 8) * g.nt : g.ng * pa::NR;                  // call rows per KV head
        g.srows = (size_t) g.ng * g.nkv * pa::NR; g.crows = (size_t) g.nkv * g.rows;
        g.qs_b = al(g.srows * pa::HD * 2); g.q_b = al(g.crows * pa::HD * 4); g.oc_b = al(g.crows * (pa::HD + 2) * 4);
        g.os_b = al(g.srows * (pa::HD + 2) * 4);
        return g;
    }

    bool start(const pa::page * pages, const uint32_t * nkeys, int n_pages, const uint16_t * Qs, const pa::config_req & cfg,
               int ng) {
        const call_geom g = geom_of(cfg, ng, ntok_hint);
        nkv_ = g.nkv; ng_ = g.ng; nt_ = g.nt; last_rows_ = g.rows;
        if (!ensure(g.dev_bytes(), g.host_bytes())) return false;   // (a growth drops the armed graph: it names the buffers)
        const bool hit = armed_match(pages, nkeys, n_pages, cfg, ng, g.nt);
        if (!hit) disarm();                                          // the stream is idle: the previous call has ended
        if (!upload_rows(pages, nkeys, n_pages, cfg.rs)) return false;
        std::memcpy(hbuf_, Qs, g.srows * pa::HD * 2);
        hout_ = (const float *) (hbuf_ + g.qs_b);
        if (hit) {                                                   // the armed launch sequence, timed as a whole
            const bool ok = hipEventRecord(e0_, st_) == hipSuccess && hipGraphLaunch(armed_.exec, st_) == hipSuccess &&
                            hipEventRecord(e1_, st_) == hipSuccess;
            armed_.used = true;                                      // one call per arm; destroyed once the stream is
                                                                     // idle (the next arm / call / page free)
            if (!ok) return fail("armed graph launch");
            n_armed_hits_++;
            return true;
        }
        (void) pa_hip_ws_set_chunk_keys(ws_, cfg.gpu_chunk);
        return enqueue(pages, nkeys, n_pages, cfg, g, true);
    }

    // the call's launch sequence on the engine stream (the query is in hbuf_); `timed` records e0 / e1 around the
    // attention (not inside a capture: the armed path times its whole graph instead)
    bool enqueue(const pa::page * pages, const uint32_t * nkeys, int n_pages, const pa::config_req & cfg, const call_geom & g,
                 bool timed) {
        char * d = dbuf_;
        uint16_t * dqs = (uint16_t *) d; float * dq = (float *) (d + g.qs_b);
        float * dO = (float *) (d + g.qs_b + g.q_b), * dm = dO + g.crows * pa::HD, * dl = dm + g.crows;
        float * sO = (float *) (d + g.qs_b + g.q_b + g.oc_b), * sm = sO + g.srows * pa::HD, * sl = sm + g.srows;
        if (hipMemcpyAsync(dqs, hbuf_, g.srows * pa::HD * 2, hipMemcpyHostToDevice, st_) != hipSuccess) return fail("Q upload");
        if (pa_hip_pack_q(dqs, g.ng, g.nkv, pa::NR, pa::HD, g.nt, dq, st_) != 0) return fail(std::string("pa_hip_pack_q: ") + pa_hip_last_error());
        std::vector<const void *> kp(n_pages), vp(n_pages);
        for (int i = 0; i < n_pages; i++) { kp[i] = pages[i].hk; vp[i] = pages[i].hv; }
        const pa_hip_shape s = {g.nkv, g.rows, (uint32_t) pa::HD, cfg.is_q8, cfg.rs, cfg.hb, PA_QMODE_F16, 1.0f};
        if (timed && hipEventRecord(e0_, st_) != hipSuccess) return fail("event");
        if (pa_hip_attn(ws_, &s, kp.data(), vp.data(), nkeys, n_pages, dq, dO, dm, dl, st_) != 0)
            return fail(std::string("pa_hip_attn: ") + pa_hip_last_error());
        if (timed && hipEventRecord(e1_, st_) != hipSuccess) return fail("event");
        if (pa_hip_unpack_rows(dO, dm, dl, g.ng, g.nkv, pa::NR, pa::HD, g.nt, sO, sm, sl, st_) != 0)
            return fail(std::string("pa_hip_unpack_rows: ") + pa_hip_last_error());
        if (hipMemcpyAsync(hbuf_ + g.qs_b, sO, g.srows * (pa::HD + 2) * 4, hipMemcpyDeviceToHost, st_) != hipSuccess)
            return fail("O download");
        return true;
    }

    // the armed graph is for exactly these pages, key counts, tokens and row format, one group
    bool armed_match(const pa::page * pages, const uint32_t * nkeys, int n_pages, const pa::config_req & cfg, int ng,
                     uint32_t nt) const {
        if (!armed_.exec || armed_.used || ng != 1 || (int) armed_.hk.size() != n_pages || armed_.nt != nt || armed_.rs != cfg.rs ||
            armed_.hb != cfg.hb || armed_.is_q8 != cfg.is_q8 || armed_.nkv != cfg.n_head_kv || armed_.chunk != cfg.gpu_chunk)
            return false;
        for (int i = 0; i < n_pages; i++) if (armed_.hk[i] != pages[i].hk || armed_.nkeys[i] != nkeys[i]) return false;
        return true;
    }
    void disarm() {
        if (armed_.exec) (void) hipGraphExecDestroy(armed_.exec);
        armed_ = armed_t();
    }

    double finish(float * O, float * m, float * l) {
        const size_t srows = (size_t) ng_ * nkv_ * pa::NR, qn = srows * pa::HD;
        if (!idle(wait_ms())) {
            for (size_t i = 0; i < qn; i++) O[i] = 0.0f;
            for (size_t i = 0; i < srows; i++) { m[i] = -INFINITY; l[i] = 0.0f; }
            return -1.0;
        }
        std::memcpy(O, hout_, qn * 4);
        std::memcpy(m, hout_ + qn, srows * 4);
        std::memcpy(l, hout_ + qn + srows, srows * 4);
        float ms = 0.0f;
        (void) hipEventElapsedTime(&ms, e0_, e1_);
        last_ms_ = ms;
        return ms;
    }
    void leave() {
        {
            std::lock_guard<std::mutex> lk(gate_mu_);
            in_call_ = false;
        }
        gate_cv_.notify_all();
    }
    static int wait_ms() {
        static const int v = [] { const char * e = getenv("PA_HIP_WAIT_MS"); const int x = e ? atoi(e) : 0; return x > 0 ? x : 30000; }();
        return v;
    }
    // the engine's stream has finished its work (bounded wait); false on a stream error or after the limit
    bool idle(int timeout_ms) {
        if (pa_hip_stream_wait(st_, timeout_ms) == 0) return true;
        return fail(std::string("engine stream: ") + pa_hip_last_error());
    }

    // the page engine the server reports TRUNCATE / CONFIG to; it takes no keys (ready() = 0), builds nothing
    struct tracker : pa::page_engine {
        hip_engine * e = nullptr;
        uint32_t page_keys() const override { return 1u << 31; }        // no page ever completes
        void configure(const pa::config_req &) override { e->on_configure(); }
        void queue(uint32_t, uint32_t, const std::vector<pa::page> &) override {}
        void truncate(uint32_t n) override { e->on_truncate(n); }
        uint32_t ready(uint32_t, uint32_t) override { return 0; }
        bool run(uint32_t, uint32_t, const uint16_t *, float *, float *, float *) override { return false; }
        std::string describe() override { return "hip engine row tracker (no page models)"; }
    };
    struct held { uint32_t key0 = 0, rows = 0; bool placed = false; };   // the HBM copy holds rows [0, rows)

    void on_configure() {
        std::lock_guard<std::mutex> lk(mu_);
        tracked_ = true;
        for (auto & x : held_) x.second = held();
    }
    void on_truncate(uint32_t n) {
        std::lock_guard<std::mutex> lk(mu_);
        for (auto & x : held_) {
            held & h = x.second;
            if (h.placed && h.key0 + h.rows > n) h.rows = n > h.key0 ? n - h.key0 : 0;
        }
    }
    // copy rows [held, nkeys) of each page (all rows [0, nkeys) while untracked); the call's pages start at key 0
    // (the tracker gives no pages to a page engine, so the server's a0 is 0: page i holds keys [i*PAGE, (i+1)*PAGE))
    bool upload_rows(const pa::page * pages, const uint32_t * nkeys, int n_pages, uint32_t rs) {
        std::lock_guard<std::mutex> lk(mu_);
        for (int i = 0; i < n_pages; i++) {
            held & h = held_[pages[i].hk];
            h.key0 = (uint32_t) i * pa::PAGE; h.placed = true;
            const uint32_t from = tracked_ ? std::min(h.rows, nkeys[i]) : 0;
            if (nkeys[i] > from) {
                const size_t off = (size_t) from * rs, b = (size_t) (nkeys[i] - from) * rs;
                if (hipMemcpyAsync((char *) pages[i].hk + off, pages[i].k + off, b, hipMemcpyHostToDevice, st_) != hipSuccess ||
                    hipMemcpyAsync((char *) pages[i].hv + off, pages[i].v + off, b, hipMemcpyHostToDevice, st_) != hipSuccess)
                    return fail("page row upload");
                rows_up_ += nkeys[i] - from;
            }
            if (tracked_) h.rows = std::max(h.rows, nkeys[i]);
        }
        return true;
    }
    static size_t al(size_t b) { return (b + 255) / 256 * 256; }
    bool ensure(size_t dev_b, size_t host_b) {
        if (dev_b <= dcap_ && host_b <= hcap_) return true;
        if (!idle(wait_ms())) return false;
        disarm();                                                    // it names the buffers freed here
        (void) hipFree(dbuf_); (void) hipHostFree(hbuf_);
        dbuf_ = nullptr; hbuf_ = nullptr; dcap_ = hcap_ = 0;
        if (hipMalloc((void **) &dbuf_, dev_b) != hipSuccess) return fail("hipMalloc call buffers");
        if (hipHostMalloc((void **) &hbuf_, host_b, hipHostMallocDefault) != hipSuccess) return fail("hipHostMalloc call buffers");
        dcap_ = dev_b; hcap_ = host_b;
        return true;
    }
    bool fail(const std::string & why) { error = why; return false; }

    pa_hip_ws * ws_ = nullptr;
    hipStream_t st_ = nullptr;
    hipEvent_t e0_ = nullptr, e1_ = nullptr;
    char * dbuf_ = nullptr, * hbuf_ = nullptr;
    size_t dcap_ = 0, hcap_ = 0;
    const float * hout_ = nullptr;
    uint32_t nkv_ = 0, ng_ = 1, nt_ = 0, last_rows_ = 0;
    double last_ms_ = 0.0;
    tracker tracker_;
    std::mutex mu_;
    std::unordered_map<void *, held> held_;   // per page (keyed by its HBM K copy)
    struct armed_t {                          // the graph arm() captured, and the call it is for
        hipGraphExec_t exec = nullptr;
        std::vector<void *> hk;
        std::vector<uint32_t> nkeys;
        uint32_t rs = 0, hb = 0, is_q8 = 0, nkv = 0, chunk = 0, nt = 0;
        bool used = false;                    // launched by a call: kept until the stream is idle, never matched again
    } armed_;
    uint64_t n_armed_ = 0, n_armed_hits_ = 0, n_warm_ = 0;
    std::mutex gate_mu_;                      // close(): no call in flight, none started after it
    std::condition_variable gate_cv_;
    bool closing_ = false, in_call_ = false;
    bool tracked_ = false;
    uint64_t rows_up_ = 0;
};

}  // namespace pa_hip_server
