// pa_hip_serve.cpp - the reference's phone-attn server on Linux with the HIP engine: pa::server (phone-attn.h:241-739,
// unchanged) constructed with a pa_hip_server::hip_engine, as pa-tool's `serve` mode constructs it with the Metal engine
// (pa-tool.cpp:54-68), and the engine's row tracker in the server's page-engine slot (its TRUNCATE / CONFIG notices). The
// unchanged pa-tool client (`pa-tool test HOST PORT ... gpu_permille=1000`) then drives the GPU over the PATN wire:
// CONFIG, APPEND into the engine's pages, ATTN / ATTN_BIG, TRUNCATE, STATS.
//
//   pa-hip-serve [port] [threads]
//
// SIGTERM / SIGINT end the process with a normal exit (exit handlers run, so a profiler wrapping the server writes its
// results). Before it exits, the engine refuses new calls and the one in flight (if any) runs to its end, and the sme_*
// calls of the server's CPU-engine pages (libpa_hip.so also exports that C ABI) are closed the same way, each wait
// bounded (PA_HIP_WAIT_MS): no HIP call is still running when the exit handlers tear the runtime down. A session in
// progress then gets error replies. Built by backburner_amd/build.py where the reference checkout (phone-attn.h) is
// present.
#include "phone-attn.h"
#include "pa_hip_engine.h"

#include <atomic>
#include <chrono>
#include <csignal>
#include <cstdio>
#include <cstdlib>
#include <thread>

static std::atomic<int> g_stop{0};   // 1: a signal asked to stop; 2: the server loop ended

static void on_signal(int) { g_stop.store(1); }

int main(int argc, char ** argv) {
    const int port = argc > 1 ? atoi(argv[1]) : pa::DEFAULT_PORT;
    const int thr = argc > 2 ? atoi(argv[2]) : 2;
    pa_hip_server::hip_engine eng;
    if (!eng.init()) {
        fprintf(stderr, "HIP engine: %s\n", eng.error.c_str());
        return 1;
    }
    pa::status st;
    pa::server srv(&st, [](const std::string & s) { fprintf(stderr, "%s\n", s.c_str()); }, thr, &eng);
    srv.set_page_engine(eng.row_tracker());   // TRUNCATE / CONFIG notices: the engine uploads only new rows
    std::signal(SIGTERM, on_signal);
    std::signal(SIGINT, on_signal);
    std::thread([&] {
        fprintf(stderr, "%s\n", srv.serve(port).c_str());
        g_stop.store(2);
    }).detach();
    while (g_stop.load() == 0) std::this_thread::sleep_for(std::chrono::milliseconds(20));
    const char * e = getenv("PA_HIP_WAIT_MS");
    const int limit = e && atoi(e) > 0 ? atoi(e) : 30000;
    const bool eng_idle = eng.close(limit);
    const bool sme_idle = pa_hip_shutdown(limit) == 0;
    if (!eng_idle || !sme_idle)
        fprintf(stderr, "pa-hip-serve: exiting with GPU work still running (%s)\n", eng_idle ? pa_hip_last_error() : eng.error.c_str());
    std::exit(g_stop.load() == 2 ? 1 : 0);   // the serving thread stays blocked in accept() or in its session
}
