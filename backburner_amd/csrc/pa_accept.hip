// pa_accept.hip - fused greedy acceptance of a draft block (the verify step's tail).
//
// No reference code exists for this in the checkout (the fork's LLAMA_BATCHED_ARGMAX, scripts/serve.sh:8-9, 281, and
// block verification, serve.sh:300-302). Semantics: a_i = argmax_j logits[i][j] with the lowest index on ties (numpy's
// rule, which also makes the first NaN win); k = the longest prefix with a_i == draft_i (i < n_rows-1); bonus = a_k.
//
// Layout: n_rows x splits workgroups, each scans one contiguous slice of one row with 16-byte loads and reduces a 64-bit
// key (orderable value << 32 | ~index) so that one unsigned max picks the largest value and, among equal values, the
// lowest index. Each workgroup publishes its key; the last one to finish (device-scope counter, no waiting) folds the
// row keys and computes (k, bonus). The counter is reset by that last workgroup, so no memset is needed between calls.
// Only that workgroup acquires at device scope (an L2 invalidate); the others only release their key.
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
    const int64_t seg = ((a.vocab + a.splits - 1) / a.splits + 3) / 4 * 4;
    const int64_t j0 = (int64_t) sp * seg, j1 = min(a.vocab, j0 + seg);
    const float * x = a.logits + (size_t) row * (size_t) a.vocab;
    unsigned long long best = 0;
    const int t = threadIdx.x;
    if ((a.vocab & 3) == 0) {
        for (int64_t j = j0 + 4 * t; j < j1; j += 4 * 256) {
            const pa_f4 v = *(const pa_f4 *) (x + j);
            best = umax64(best, accept_key(v[0], (uint32_t) j));
            best = umax64(best, accept_key(v[1], (uint32_t) (j + 1)));
            best = umax64(best, accept_key(v[2], (uint32_t) (j + 2)));
            best = umax64(best, accept_key(v[3], (uint32_t) (j + 3)));
        }
    } else {
        for (int64_t j = j0 + t; j < j1; j += 256) best = umax64(best, accept_key(x[j], (uint32_t) j));
    }
    for (int off = 32; off > 0; off >>= 1) best = umax64(best, __shfl_xor(best, off));
    if ((t & 63) == 0) red[t / 64] = best;
    __syncthreads();
    if (t == 0) {
        best = umax64(umax64(red[0], red[1]), umax64(red[2], red[3]));
        __hip_atomic_store(&a.part[row * a.splits + sp], best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // release at device scope (one L2 write-back); only the completing workgroup acquires (invalidates)
        const unsigned int done = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        last = done == (unsigned int) (a.n_rows * a.splits - 1);
    }
    __syncthreads();
    if (!last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // the last workgroup: fold each row's keys, then the accepted prefix
    __shared__ int32_t am[64];
    if (t < a.n_rows) {
        unsigned long long b = 0;
        for (int s = 0; s < a.splits; s++)
            b = umax64(b, __hip_atomic_load(&a.part[t * a.splits + s], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        am[t] = (int32_t) (0xffffffffu - (uint32_t) (b & 0xffffffffu));
    }
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
