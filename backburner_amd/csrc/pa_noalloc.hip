// pa_noalloc.hip - pa_hip_attn_noalloc: the engine path's partial attention for callers that cannot allocate device
// memory (code under HIP graph capture, serving loops that forbid hipMalloc). No counterpart in the reference.
//
// The call's split-K slots go to `scratch`, a fixed device array of PA_HIP_NOALLOC_SCRATCH bytes that every GPU the
// library runs on holds from its first such call until the process ends. The array's name is a host-side stand-in in
// host code; its device address is looked up once per device (hipGetSymbolAddress, with that device current) and only
// that address is passed to the kernels. Every call on one GPU shares that GPU's array: calls that overlap on one GPU
// (different streams, or without ordering) race on it. Nothing in it needs to start at zero - each slot is written by
// its workgroup before the merge reads it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/phone_attn_hip.h"
#include "pa_attn.h"

static __device__ __align__(256) char scratch[PA_HIP_NOALLOC_SCRATCH];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
char * g_scratch[MAX_DEVICES] = {};   // the device address of `scratch` on each device, once looked up

// the current device's copy of the array (looked up on the device's first call), or null with the error set
char * device_scratch() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
        (void) hipGetLastError();
        pa_hip::set_error("pa_hip_attn_noalloc: no current HIP device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_scratch[dev]) {
        void * p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void) hipGetLastError();
            pa_hip::set_error(std::string("pa_hip_attn_noalloc: hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
            return nullptr;
        }
        g_scratch[dev] = (char *) p;
    }
    return g_scratch[dev];
}

}  // namespace

extern "C" int pa_hip_attn_noalloc(const pa_hip_shape * shape, const void * const * k_pages, const void * const * v_pages,
                                   const uint32_t * nkeys, int n_pages, const float * Q, float * O, float * m, float * l,
                                   void * stream) {
    char * p = device_scratch();
    if (!p) return -1;
    return pa_hip::attn_fixed_scratch(p, PA_HIP_NOALLOC_SCRATCH, shape, k_pages, v_pages, nkeys, n_pages, Q, O, m, l,
                                      (hipStream_t) stream);
}
