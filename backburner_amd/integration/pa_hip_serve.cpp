// pa_hip_serve.cpp - the reference's phone-attn server on Linux with the HIP engine: pa::server (phone-attn.h:241-739,
// unchanged) constructed with a pa_hip_server::hip_engine, as pa-tool's `serve` mode constructs it with the Metal engine
// (pa-tool.cpp:54-68). The unchanged pa-tool client (`pa-tool test HOST PORT ... gpu_permille=1000`) then drives the
// GPU over the PATN wire: CONFIG, APPEND into the engine's pages, ATTN / ATTN_BIG, TRUNCATE, STATS.
//
//   pa-hip-serve [port] [threads]
//
// Built by oracle/Makefile where the reference checkout (phone-attn.h) is present; the server's non-GPU pages go to the
// sme_* C ABI, which libpa_hip.so also exports.
#include "phone-attn.h"
#include "pa_hip_engine.h"

#include <cstdio>
#include <cstdlib>

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
    fprintf(stderr, "%s\n", srv.serve(port).c_str());
    return 1;
}
