// pa_pack.hip - the row layout between the reference server's engine calls and a pa_hip_attn call, on the device.
//
// The server hands its GPU engine ng groups of 8 tokens (pa::engine::begin, phone-attn.h:174-176):
//   Qs = f16(q*scale) [ng][nkv][nr][hd], row i of a head = GQA member i / 8, token i % 8,
// and wants (O, m, l) back as [ng][nkv*nr] rows. A pa_hip_attn call runs on fp32 Q [nkv][rows][hd]:
//   - the groups back to back per KV head (rows = ng*nr, row g*nr + i), or
//   - for one group with 1 <= ntok < 8 real tokens, only the real rows (rows = (nr/8)*ntok, member k's token t at
//     k*ntok + t), as the reference's Metal engine packs them (pa-metal.mm:630-634 geom, 661-672 pack_q).
// pa_pack_q_kernel converts and places Q; pa_unpack_kernel places (O, m, l) back, giving the rows of tokens the call
// did not have (0, -inf, 0): no keys (pa-metal.mm:501-505). pa_warm_kernel is the server's keep-warm dispatch between
// calls (the Metal engine's 32-thread warm dispatch, pa-metal.mm:955-968).
#include <hip/hip_runtime.h>

#include <cmath>
#include <string>

#include "../../include/phone_attn_hip.h"
#include "pa_attn.h"
#include "pa_common.h"

namespace {

constexpr uint32_t TOK = 8;   // tokens per group of the server's query rows

struct PackGeom {
    uint32_t ng, nkv, nr, hd, nt, rows;   // rows = call rows per KV head
    // the server row (group g, row i of the head) of call row r
    __device__ __forceinline__ void src(uint32_t r, uint32_t & g, uint32_t & i) const {
        if (nt) { g = 0; i = (r / nt) * TOK + r % nt; }
        else { g = r / nr; i = r % nr; }
    }
};

// one thread per 4 consecutive values of a row (hd is a multiple of 4)
__global__ __launch_bounds__(256) void pa_pack_q_kernel(const uint16_t * qs, float * q, PackGeom p) {
    const uint32_t hq = p.hd / 4;
    const uint64_t n = (uint64_t) p.nkv * p.rows * hq;
    for (uint64_t x = (uint64_t) blockIdx.x * 256 + threadIdx.x; x < n; x += (uint64_t) gridDim.x * 256) {
        const uint32_t d4 = (uint32_t) (x % hq);
        const uint64_t rr = x / hq;
        const uint32_t r = (uint32_t) (rr % p.rows), h = (uint32_t) (rr / p.rows);
        uint32_t g, i;
        p.src(r, g, i);
        const pa_h4 v = *(const pa_h4 *) (qs + (((uint64_t) g * p.nkv + h) * p.nr + i) * p.hd + 4 * d4);
        *(float4 *) (q + rr * p.hd + 4 * d4) = make_float4((float) v[0], (float) v[1], (float) v[2], (float) v[3]);
    }
}

__global__ __launch_bounds__(256) void pa_unpack_kernel(const float * O, const float * m, const float * l, float * Os,
                                                        float * ms, float * ls, PackGeom p) {
    const uint32_t hq = p.hd / 4;
    const uint64_t n = (uint64_t) p.ng * p.nkv * p.nr * hq;
    for (uint64_t x = (uint64_t) blockIdx.x * 256 + threadIdx.x; x < n; x += (uint64_t) gridDim.x * 256) {
        const uint32_t d4 = (uint32_t) (x % hq);
        const uint64_t R = x / hq;                                // server row: group g, head h, row i
        const uint32_t i = (uint32_t) (R % p.nr), h = (uint32_t) ((R / p.nr) % p.nkv), g = (uint32_t) (R / ((uint64_t) p.nr * p.nkv));
        float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float mv = -INFINITY, lv = 0.0f;
        if (!p.nt || i % TOK < p.nt) {
            const uint32_t r = p.nt ? (i / TOK) * p.nt + i % TOK : g * p.nr + i;
            const uint64_t sr = (uint64_t) h * p.rows + r;
            o = *(const float4 *) (O + sr * p.hd + 4 * d4);
            mv = m[sr];
            lv = l[sr];
        }
        *(float4 *) (Os + R * p.hd + 4 * d4) = o;
        if (d4 == 0) { ms[R] = mv; ls[R] = lv; }
    }
}

bool geom(const char * fn, uint32_t ng, uint32_t nkv, uint32_t nr, uint32_t hd, uint32_t ntok, PackGeom & p) {
    if (ng == 0 || nkv == 0 || nr == 0 || nr % TOK || hd == 0 || hd % 4 || ntok > TOK || (ntok && ntok < TOK && ng != 1)) {
        pa_hip::set_error(std::string(fn) + ": bad geometry (ng " + std::to_string(ng) + ", nkv " + std::to_string(nkv) +
                          ", nr " + std::to_string(nr) + " (a multiple of 8), hd " + std::to_string(hd) +
                          " (a multiple of 4), ntok " + std::to_string(ntok) + " (0..8; below 8 only with one group))");
        return false;
    }
    if ((uint64_t) ng * nkv * nr * hd >= (1ull << 40)) { pa_hip::set_error(std::string(fn) + ": too many rows"); return false; }
    p.ng = ng; p.nkv = nkv; p.nr = nr; p.hd = hd;
    p.nt = (ntok >= 1 && ntok < TOK) ? ntok : 0;
    p.rows = p.nt ? (nr / TOK) * p.nt : ng * nr;
    return true;
}

uint32_t grid_of(uint64_t n) { return (uint32_t) std::min<uint64_t>((n + 255) / 256, 8192); }

bool launched(const char * fn) {
    const hipError_t e = hipGetLastError();
    if (e == hipSuccess) return true;
    pa_hip::set_error(std::string(fn) + ": launch: " + hipGetErrorString(e));
    return false;
}

// one wave that reads nothing and writes nothing: a dispatch that keeps the device's clocks up between calls
__global__ __launch_bounds__(64) void pa_warm_kernel(uint32_t * sink, uint32_t v) {
    if (sink && v == 0xffffffffu && threadIdx.x == 0) *sink = v;   // never true: the host passes a null sink
}

}  // namespace

extern "C" int pa_hip_warm(void * stream) {
    hipLaunchKernelGGL(pa_warm_kernel, dim3(1), dim3(64), 0, (hipStream_t) stream, (uint32_t *) nullptr, 0u);
    return launched("pa_hip_warm") ? 0 : -1;
}

extern "C" int pa_hip_pack_q(const uint16_t * qs, uint32_t ng, uint32_t nkv, uint32_t nr, uint32_t hd, uint32_t ntok,
                             float * q, void * stream) {
    PackGeom p;
    if (!geom("pa_hip_pack_q", ng, nkv, nr, hd, ntok, p)) return -1;
    if (!qs || !q || ((uintptr_t) qs & 7) || ((uintptr_t) q & 15)) {
        pa_hip::set_error("pa_hip_pack_q: qs must be 8-byte and q 16-byte aligned device pointers");
        return -1;
    }
    hipLaunchKernelGGL(pa_pack_q_kernel, dim3(grid_of((uint64_t) p.nkv * p.rows * (hd / 4))), dim3(256), 0,
                       (hipStream_t) stream, qs, q, p);
    return launched("pa_hip_pack_q") ? 0 : -1;
}

extern "C" int pa_hip_unpack_rows(const float * O, const float * m, const float * l, uint32_t ng, uint32_t nkv, uint32_t nr,
                                  uint32_t hd, uint32_t ntok, float * Os, float * ms, float * ls, void * stream) {
    PackGeom p;
    if (!geom("pa_hip_unpack_rows", ng, nkv, nr, hd, ntok, p)) return -1;
    if (!O || !m || !l || !Os || !ms || !ls || ((uintptr_t) O & 15) || ((uintptr_t) Os & 15)) {
        pa_hip::set_error("pa_hip_unpack_rows: null argument, or O / Os not 16-byte aligned");
        return -1;
    }
    hipLaunchKernelGGL(pa_unpack_kernel, dim3(grid_of((uint64_t) ng * nkv * nr * (hd / 4))), dim3(256), 0,
                       (hipStream_t) stream, O, m, l, Os, ms, ls, p);
    return launched("pa_hip_unpack_rows") ? 0 : -1;
}
