// pa_accept.hip - fused greedy acceptance of a draft block (the verify step's tail).
//
// No reference code exists for this in the checkout (the fork's LLAMA_BATCHED_ARGMAX, scripts/serve.sh:8-9, 281, and
// block verification, serve.sh:300-302). Semantics: a_i = argmax_j logits[i][j] with the lowest index on ties (numpy's
// rule, which also makes the first NaN win); k = the longest prefix with a_i == draft_i (i < n_rows-1); bonus = a_k.
//
// Layout: n_rows x splits workgroups; workgroup (row, sp) scans values [S sp, S sp + S) of its row (S = ACCEPT_SEG),
// every thread issuing all its loads at once (S / 1024 16-byte loads, or S / 256 scalar ones when the vocab is not a
// multiple of 4), and reduces a 64-bit key (orderable value << 32 | ~index) so that one unsigned max picks the largest value
// and, among equal values, the lowest index. Each workgroup publishes its key with a write-through store and waits for
// it to complete before it counts itself done on a device-scope counter; the last one reads the keys with
// write-through loads, folds them per row and computes (k, bonus). No cache write-back or invalidate is needed: the
// keys never sit in an XCD's L2. The last workgroup resets the counter, so no memset is needed between calls.
#include "pa_attn.h"
#include "pa_common.h"

namespace pa_hip {

__device__ __forceinline__ unsigned long long accept_key(float x, uint32_t idx) {
    uint32_t u = __builtin_bit_cast(uint32_t, x);
    uint32_t k;
    if (x != x) k = 0xffffffffu;                 // NaN above everything (numpy.argmax returns the first NaN)
    else {
        if (u == 0x80000000u) u = 0u;            // -0 == +0
        k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    }
    return ((unsigned long long) k << 32) | (unsigned long long) (0xffffffffu - idx);
}


__device__ __forceinline__ unsigned long long umax64(unsigned long long a, unsigned long long b) { return a > b ? a : b; }

__global__ __launch_bounds__(256) void accept_kernel(const AcceptArgs a) {
    __shared__ unsigned long long red[4];
    __shared__ bool last;
    const int row = blockIdx.x / a.splits, sp = blockIdx.x % a.splits;
    const int64_t j0 = (int64_t) sp * ACCEPT_SEG, j1 = min(a.vocab, j0 + ACCEPT_SEG);
    const float * x = a.logits + (size_t) row * (size_t) a.vocab;
    unsigned long long best = 0;
    const int t = threadIdx.x;
    if ((a.vocab & 3) == 0) {                                        // j < j1 implies j + 3 < vocab
        constexpr int NU = ACCEPT_SEG / 1024;
        pa_f4 v[NU];
        #pragma unroll
        for (int u = 0; u < NU; u++) {
            const int64_t j = j0 + 4 * t + 1024 * u;
            v[u] = j < j1 ? *(const pa_f4 *) (x + j) : (pa_f4){0.f, 0.f, 0.f, 0.f};
        }
        #pragma unroll
        for (int u = 0; u < NU; u++) {
            const int64_t j = j0 + 4 * t + 1024 * u;
            if (j < j1) {
                #pragma unroll
                for (int e = 0; e < 4; e++) best = umax64(best, accept_key(v[u][e], (uint32_t) (j + e)));
            }
        }
    } else {
        constexpr int NU = ACCEPT_SEG / 256;
        float v[NU];
        #pragma unroll
        for (int u = 0; u < NU; u++) {
            const int64_t j = j0 + t + 256 * u;
            v[u] = j < j1 ? x[j] : 0.0f;
        }
        #pragma unroll
        for (int u = 0; u < NU; u++) {
            const int64_t j = j0 + t + 256 * u;
            if (j < j1) best = umax64(best, accept_key(v[u], (uint32_t) j));
        }
    }
    for (int off = 32; off > 0; off >>= 1) best = umax64(best, __shfl_xor(best, off));
    if ((t & 63) == 0) red[t / 64] = best;
    __syncthreads();
    if (t == 0) {
        best = umax64(umax64(red[0], red[1]), umax64(red[2], red[3]));
        // write-through store (device scope), complete before the count below is made
        __hip_atomic_store(&a.part[row * a.splits + sp], best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        const unsigned int done = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = done == (unsigned int) (a.n_rows * a.splits - 1);
    }
    __syncthreads();
    if (!last) return;
    // the last workgroup: every thread reads a share of all keys at once (write-through loads) and folds them into
    // its row's slot (LDS atomic max), then the accepted prefix
    __shared__ unsigned long long rk[64];
    __shared__ int32_t am[64];
    if (t < a.n_rows) rk[t] = 0;
    __syncthreads();
    const int nk = a.n_rows * a.splits;
    for (int i0 = 0; i0 < nk; i0 += 4 * 256) {
        unsigned long long k4[4];
        #pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = i0 + t + 256 * u;
            k4[u] = i < nk ? __hip_atomic_load(&a.part[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
        }
        #pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = i0 + t + 256 * u;
            if (i < nk) __hip_atomic_fetch_max(&rk[i / a.splits], k4[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }
    __syncthreads();
    if (t < a.n_rows) am[t] = (int32_t) (0xffffffffu - (uint32_t) (rk[t] & 0xffffffffu));
    __syncthreads();
    if (t == 0) {
        int k = 0;
        while (k < a.n_rows - 1 && am[k] == a.draft[k]) k++;
        a.out[0] = k;
        a.out[1] = am[k];
        __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (t < a.n_rows) a.out[2 + t] = am[t];
}

hipError_t launch_accept(const AcceptArgs & a, hipStream_t st) {
    hipLaunchKernelGGL(accept_kernel, dim3((uint32_t) (a.n_rows * a.splits)), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace pa_hip
