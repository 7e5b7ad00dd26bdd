// pa_hip_engine.h - the GPU engine of the reference's phone-attn server on an MI355X: a pa::engine (phone-attn.h:166-183,
// the interface the Metal engine implements in pa-metal.mm:674-953) over libpa_hip.so's pa_hip_attn.
//
// Include phone-attn.h first. One call = one pa_hip_attn launch sequence over the call's pages, on the engine's stream:
//   begin()  Qs = f16(q*scale) [ng][nkv][NR][HD] -> fp32 [nkv][ng*NR][HD] (exact) in PA_QMODE_F16 with scale 1, the
//            pages' rows into their HBM copies, the launch, the copy back of (O, m, l); nothing waits
//   end()    waits, reorders (O, m, l) to the server's [ng][nkv*NR] rows; returns the attention's GPU ms
// Pages: the unchanged server writes received rows into page.k / page.v with memcpy (store_rows, phone-attn.h:305-319),
// so they are pinned host memory; page.hk / page.hv are their HBM copies, which begin() refreshes for the rows the
// call reads (every held row: the engine cannot see a TRUNCATE that rewrites rows in place). A server that stores
// APPEND rows on the device itself (pa_hip_append_rows) reads the HBM pages with no copy.
// Failure: begin() returns false (the server answers "GPU engine failed to start"); end() returns -1 with
// O = 0, m = -inf, l = 0, the Metal engine's failure value (pa-metal.mm:932-937).
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>
#include <string>
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
        return true;
    }
    ~hip_engine() override {
        if (st_) (void) hipStreamSynchronize(st_);
        if (ws_) pa_hip_ws_destroy(ws_);
        (void) hipFree(dbuf_);
        (void) hipHostFree(hbuf_);
        if (e0_) (void) hipEventDestroy(e0_);
        if (e1_) (void) hipEventDestroy(e1_);
        if (st_) (void) hipStreamDestroy(st_);
    }

    bool alloc_page(size_t bytes, pa::page & p) override {
        void * k = nullptr, * v = nullptr, * hk = nullptr, * hv = nullptr;
        if (hipHostMalloc(&k, bytes, hipHostMallocDefault) != hipSuccess) return false;
        if (hipHostMalloc(&v, bytes, hipHostMallocDefault) != hipSuccess) { (void) hipHostFree(k); return false; }
        if (pa_hip_alloc_page(bytes, &hk, &hv) != 0) { (void) hipHostFree(k); (void) hipHostFree(v); return false; }
        p.k = (uint8_t *) k; p.v = (uint8_t *) v; p.hk = hk; p.hv = hv;
        return true;
    }
    void free_page(pa::page & p) override {
        (void) hipStreamSynchronize(st_);                            // no copy of this page in flight
        (void) hipHostFree(p.k); (void) hipHostFree(p.v);
        pa_hip_free_page(p.hk, p.hv);
        p = pa::page();
    }

    bool begin(const pa::page * pages, const uint32_t * nkeys, int n_pages, const uint16_t * Qs, const pa::config_req & cfg,
               int ng) override {
        nkv_ = (int) cfg.n_head_kv; ng_ = ng;
        const size_t rows = (size_t) ng * nkv_ * pa::NR, qn = rows * pa::HD;
        const size_t need = (2 * qn + 2 * rows) * sizeof(float);      // device: Q, O, m, l; host: the same
        if (need > cap_) {
            (void) hipStreamSynchronize(st_);
            (void) hipFree(dbuf_); (void) hipHostFree(hbuf_);
            dbuf_ = nullptr; hbuf_ = nullptr; cap_ = 0;
            if (hipMalloc((void **) &dbuf_, need) != hipSuccess) return fail("hipMalloc Q/O");
            if (hipHostMalloc((void **) &hbuf_, need, hipHostMallocDefault) != hipSuccess) return fail("hipHostMalloc Q/O");
            cap_ = need;
        }
        std::vector<const void *> kp(n_pages), vp(n_pages);
        for (int i = 0; i < n_pages; i++) {
            const size_t b = (size_t) nkeys[i] * cfg.rs;
            if (hipMemcpyAsync(pages[i].hk, pages[i].k, b, hipMemcpyHostToDevice, st_) != hipSuccess ||
                hipMemcpyAsync(pages[i].hv, pages[i].v, b, hipMemcpyHostToDevice, st_) != hipSuccess)
                return fail("page upload");
            kp[i] = pages[i].hk; vp[i] = pages[i].hv;
        }
        float * hq = hbuf_;
        for (int g = 0; g < ng; g++)                                 // [ng][nkv][NR][HD] -> [nkv][ng*NR][HD]
            for (int h = 0; h < nkv_; h++)
                for (int r = 0; r < pa::NR; r++) {
                    const uint16_t * src = Qs + (((size_t) g * nkv_ + h) * pa::NR + r) * pa::HD;
                    float * dst = hq + (((size_t) h * ng + g) * pa::NR + r) * pa::HD;
                    for (int d = 0; d < pa::HD; d++) dst[d] = pa::h2f(src[d]);
                }
        float * dq = dbuf_, * dO = dq + qn, * dm = dO + qn, * dl = dm + rows;
        if (hipMemcpyAsync(dq, hq, qn * sizeof(float), hipMemcpyHostToDevice, st_) != hipSuccess) return fail("Q upload");
        const pa_hip_shape s = {(uint32_t) nkv_, (uint32_t) (ng * pa::NR), (uint32_t) pa::HD, cfg.is_q8, cfg.rs, cfg.hb,
                                PA_QMODE_F16, 1.0f};
        if (hipEventRecord(e0_, st_) != hipSuccess) return fail("event");
        if (pa_hip_attn(ws_, &s, kp.data(), vp.data(), nkeys, n_pages, dq, dO, dm, dl, st_) != 0)
            return fail(std::string("pa_hip_attn: ") + pa_hip_last_error());
        if (hipEventRecord(e1_, st_) != hipSuccess ||
            hipMemcpyAsync(hbuf_ + qn, dO, (qn + 2 * rows) * sizeof(float), hipMemcpyDeviceToHost, st_) != hipSuccess)
            return fail("O download");
        return true;
    }

    double end(float * O, float * m, float * l) override {
        const size_t rows = (size_t) ng_ * nkv_ * pa::NR, qn = rows * pa::HD;
        if (hipStreamSynchronize(st_) != hipSuccess) {
            fail("hipStreamSynchronize");
            for (size_t i = 0; i < qn; i++) O[i] = 0.0f;
            for (size_t i = 0; i < rows; i++) { m[i] = -INFINITY; l[i] = 0.0f; }
            return -1.0;
        }
        const float * hO = hbuf_ + qn, * hm = hO + qn, * hl = hm + rows;
        for (int g = 0; g < ng_; g++)                                // [nkv][ng*NR] -> [ng][nkv*NR]
            for (int h = 0; h < nkv_; h++)
                for (int r = 0; r < pa::NR; r++) {
                    const size_t src = ((size_t) h * ng_ + g) * pa::NR + r, dst = ((size_t) g * nkv_ + h) * pa::NR + r;
                    for (int d = 0; d < pa::HD; d++) O[dst * pa::HD + d] = hO[src * pa::HD + d];
                    m[dst] = hm[src];
                    l[dst] = hl[src];
                }
        float ms = 0.0f;
        (void) hipEventElapsedTime(&ms, e0_, e1_);
        last_ms_ = ms;
        return ms;
    }

    double exec_ms() const override { return last_ms_; }
    std::string describe() override { return "hip MI355X (libpa_hip)"; }

private:
    bool fail(const std::string & why) { error = why; return false; }
    pa_hip_ws * ws_ = nullptr;
    hipStream_t st_ = nullptr;
    hipEvent_t e0_ = nullptr, e1_ = nullptr;
    float * dbuf_ = nullptr, * hbuf_ = nullptr;
    size_t cap_ = 0;
    int nkv_ = 0, ng_ = 1;
    double last_ms_ = 0.0;
};

}  // namespace pa_hip_server
