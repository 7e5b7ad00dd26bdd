// pa_merge.hip - the split-K merge: the partial results of a call's workgroups (one slot per workgroup: O unnormalised
// against the slot's base-2 max, the max, the sum) folded into the call's (O, m, l), or straight into the ATTN reply
// format when the call asks for it (pa_hip_attn_reply). Every fold takes M = max over the slots, gives -inf slots
// weight 0, and forms O = sum w_c O_c, L = sum w_c l_c with w_c = 2^(m_c - M).
//
// Reference roles: pa_merge / pa_merge_big (pa-metal.mm:137-159, 490-524: M = max, skip -inf slots, w = exp(m_c - M),
// O = sum w O_c, L = sum w l_c); the reply format of phone-attn.h:651-655.
#include "pa_attn.h"
#include "pa_common.h"

namespace pa_hip {

// ---------------------------------------------------------------- split-K fold as its own kernel
// The reply format of a merged row (the ATTN reply, phone-attn.h:651-655), written in place of (O, m, l) when the call
// asks for it: Oh = f16(O * (1 / L)) (0 where L = 0) for k consecutive dims, lse = M ln 2 + log L by the thread given
// `row_stats`. The same roundings as storing (O, m, l) and normalising them afterwards.
template <int K>
__device__ __forceinline__ void merge_write_reply(const MergeArgs & a, size_t off, const float * o, float M, float L, uint32_t r,
                                                  bool row_stats) {
    #pragma clang fp contract(off)
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    #pragma unroll
    for (int k = 0; k < K; k++) a.Oh[off + k] = __builtin_bit_cast(uint16_t, (_Float16) pa_f32(o[k] * inv));
    if (row_stats) {
        const float mm = M == -INFINITY ? -INFINITY : M * PA_LN2;
        a.lse[r] = L > 0.0f ? mm + logf(L) : -INFINITY;
    }
}

// More slots than one workgroup's lanes hold (calls of several launches: more than MAXP pages): one workgroup of 256
// threads per (row, 32 dims), as the wide merge below, over the slots in batches of 256 - first the max over every
// batch's (max, sum) pairs, then per batch the wide merge's loads (eight lanes per slot line, the batch's loads issued
// at once), weighed by that max and summed.
template <int HD>
__global__ __launch_bounds__(256) void merge_batched_kernel(const MergeArgs a) {
    constexpr int NQ = HD / 32, NT = 256, NWV = NT / 64;
    __shared__ float sM[NWV], sL[NWV];
    __shared__ pa_f4 sA[NWV][8];
    const uint32_t r = blockIdx.x / NQ, dq = blockIdx.x % NQ;   // output row h*rows + i, dims 32 dq .. +31
    const uint32_t h = r / a.rows, i = r % a.rows;
    const int t = threadIdx.x, lane = t % 64, wv = t / 64;
    const size_t pr = ((size_t) h * a.qr + i) * a.rst;              // slot s of the row at s * a.sst + pr
    const uint32_t nb = (a.n_slots + NT - 1) / NT;
    float M = -INFINITY;
    for (uint32_t b = 0; b < nb; b++) {
        const uint32_t s = b * NT + t;
        if (s < a.n_slots) M = fmaxf(M, a.pml[s * a.sst + pr].x);
    }
    #pragma unroll
    for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
    if (lane == 0) sM[wv] = M;
    __syncthreads();
    #pragma unroll
    for (int k = 0; k < NWV; k++) M = fmaxf(M, sM[k]);
    const float Ms = M == -INFINITY ? 0.0f : M;
    pa_f4 acc = {0.f, 0.f, 0.f, 0.f};
    float L = 0.0f;
    for (uint32_t b = 0; b < nb; b++) {
        pa_f4 o[8];
        #pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t s = b * NT + 64 * wv + lane / 8 + 8 * j;
            o[j] = s < a.n_slots ? *(const pa_f4 *) (a.po + (s * a.sst + pr) * HD + 32 * dq + 4 * (lane % 8))
                                 : (pa_f4){0.f, 0.f, 0.f, 0.f};
        }
        const uint32_t st = b * NT + t;
        const float2 ml = st < a.n_slots ? a.pml[st * a.sst + pr] : make_float2(-INFINITY, 0.0f);
        const float w = __builtin_amdgcn_exp2f(ml.x - Ms);          // -inf (an empty or absent slot) -> 0
        L += w * ml.y;
        #pragma unroll
        for (int j = 0; j < 8; j++) acc += __shfl(w, lane / 8 + 8 * j) * o[j];   // slot's weight: this wave's lane
    }
    #pragma unroll
    for (int off = 32; off > 0; off >>= 1) L += __shfl_xor(L, off);
    #pragma unroll
    for (int off = 8; off < 64; off <<= 1)
        #pragma unroll
        for (int k = 0; k < 4; k++) acc[k] += __shfl_xor(acc[k], off);
    if (lane < 8) sA[wv][lane] = acc;
    if (lane == 0) sL[wv] = L;
    __syncthreads();
    if (wv != 0 || lane >= 8) return;
    acc = sA[0][lane];
    L = sL[0];
    #pragma unroll
    for (int k = 1; k < NWV; k++) { acc += sA[k][lane]; L += sL[k]; }
    const size_t off = (size_t) r * HD + 32 * dq + 4 * lane;        // lanes 0-7 of wave 0: dims 32 dq + 4 lane .. +3
    if (a.Oh) {
        const float v[4] = {acc[0], acc[1], acc[2], acc[3]};
        merge_write_reply<4>(a, off, v, M, L, r, dq == 0 && lane == 0);
        return;
    }
    *(pa_f4 *) (a.O + off) = acc;
    if (dq == 0 && lane == 0) {
        a.m[r] = M == -INFINITY ? -INFINITY : M * PA_LN2;
        a.l[r] = L;
    }
}

// Many slots (split-K decode up to 256, verify up to 64): one workgroup of NT threads (256, or one wave for at most 64
// slots) per (row, 32 dims), every load of the fold issued at once (one memory latency, not one per slot). Lane l of
// wave v reads dims 4 (l % 8) .. +3 of slots 64 v + l / 8 + 8 j (j < 8), so that eight lanes read one slot's 128 bytes
// and a load instruction touches eight whole lines; thread t also reads slot t's (max, sum). The weights reach the
// lanes that hold a slot's dims by a shuffle, the dims' sums by xor-shuffles over the eight-lane groups, then across
// waves through LDS.
template <int HD, int NT>
__global__ __launch_bounds__(NT) void merge_wide_kernel(const MergeArgs a) {
    constexpr int NQ = HD / 32, NWV = NT / 64;
    __shared__ float sM[NWV], sL[NWV];
    __shared__ pa_f4 sA[NWV][8];
    const uint32_t r = blockIdx.x / NQ, dq = blockIdx.x % NQ;   // output row h*rows + i, dims 32 dq .. +31
    const uint32_t h = r / a.rows, i = r % a.rows;
    const int t = threadIdx.x, lane = t % 64, wv = t / 64;
    const size_t pr = ((size_t) h * a.qr + i) * a.rst;              // slot s of the row at s * a.sst + pr
    pa_f4 o[8];
    #pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t s = 64 * wv + lane / 8 + 8 * j;
        o[j] = s < a.n_slots ? *(const pa_f4 *) (a.po + (s * a.sst + pr) * HD + 32 * dq + 4 * (lane % 8))
                             : (pa_f4){0.f, 0.f, 0.f, 0.f};
    }
    const float2 ml = (uint32_t) t < a.n_slots ? a.pml[t * a.sst + pr] : make_float2(-INFINITY, 0.0f);
    float M = ml.x;
    #pragma unroll
    for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
    if constexpr (NWV > 1) {
        if (lane == 0) sM[wv] = M;
        __syncthreads();
        #pragma unroll
        for (int k = 0; k < NWV; k++) M = fmaxf(M, sM[k]);
    }
    const float Ms = M == -INFINITY ? 0.0f : M;
    const float w = __builtin_amdgcn_exp2f(ml.x - Ms);              // -inf (an empty or absent slot) -> 0
    float L = w * ml.y;
    #pragma unroll
    for (int off = 32; off > 0; off >>= 1) L += __shfl_xor(L, off);
    pa_f4 acc = {0.f, 0.f, 0.f, 0.f};
    #pragma unroll
    for (int j = 0; j < 8; j++) acc += __shfl(w, lane / 8 + 8 * j) * o[j];   // slot 64 wv + l / 8 + 8 j is this wave's lane l / 8 + 8 j
    #pragma unroll
    for (int off = 8; off < 64; off <<= 1)
        #pragma unroll
        for (int k = 0; k < 4; k++) acc[k] += __shfl_xor(acc[k], off);
    if constexpr (NWV > 1) {
        if (lane < 8) sA[wv][lane] = acc;
        if (lane == 0) sL[wv] = L;
        __syncthreads();
        if (wv != 0 || lane >= 8) return;
        acc = sA[0][lane];
        L = sL[0];
        #pragma unroll
        for (int k = 1; k < NWV; k++) { acc += sA[k][lane]; L += sL[k]; }
    } else if (lane >= 8) {
        return;
    }
    // lanes 0-7 of wave 0: dims 32 dq + 4 lane .. +3
    const size_t off = (size_t) r * HD + 32 * dq + 4 * lane;
    if (a.Oh) {
        const float v[4] = {acc[0], acc[1], acc[2], acc[3]};
        merge_write_reply<4>(a, off, v, M, L, r, dq == 0 && lane == 0);
        return;
    }
    *(pa_f4 *) (a.O + off) = acc;
    if (dq == 0 && lane == 0) {
        a.m[r] = M == -INFINITY ? -INFINITY : M * PA_LN2;
        a.l[r] = L;
    }
}

// Few slots (prefill, up to 16): 256 / (HD / 4) rows per workgroup, HD / 4 threads per row (4 dims each), every
// slot's load issued at once.
template <int HD>
__global__ __launch_bounds__(256) void merge_rows_kernel(const MergeArgs a) {
    constexpr int TPR = HD / 4, RPW = 256 / TPR, MS = 16;
    const int t = threadIdx.x, d4 = t % TPR;
    const uint32_t r = blockIdx.x * RPW + t / TPR;                   // output row h*rows + i
    if (r >= a.nkv * a.rows) return;
    const uint32_t h = r / a.rows, i = r % a.rows;
    const size_t pr = ((size_t) h * a.qr + i) * a.rst;              // slot s at s * a.sst + pr
    float2 ml[MS];
    pa_f4 o[MS];
    #pragma unroll
    for (int s = 0; s < MS; s++) {
        if ((uint32_t) s < a.n_slots) {
            ml[s] = a.pml[s * a.sst + pr];
            o[s] = *(const pa_f4 *) (a.po + (s * a.sst + pr) * HD + 4 * d4);
        } else {
            ml[s] = make_float2(-INFINITY, 0.0f);
            o[s] = (pa_f4){0.f, 0.f, 0.f, 0.f};
        }
    }
    float M = -INFINITY;
    #pragma unroll
    for (int s = 0; s < MS; s++) M = fmaxf(M, ml[s].x);
    const float Ms = M == -INFINITY ? 0.0f : M;
    pa_f4 acc = {0.f, 0.f, 0.f, 0.f};
    float L = 0.0f;
    #pragma unroll
    for (int s = 0; s < MS; s++) {
        const float w = __builtin_amdgcn_exp2f(ml[s].x - Ms);       // -inf (an empty or absent slot) -> 0
        acc += w * o[s];
        L += w * ml[s].y;
    }
    if (a.Oh) {
        const float ov[4] = {acc[0], acc[1], acc[2], acc[3]};
        merge_write_reply<4>(a, (size_t) r * HD + 4 * d4, ov, M, L, r, d4 == 0);
        return;
    }
    *(pa_f4 *) (a.O + (size_t) r * HD + 4 * d4) = acc;
    if (d4 == 0) { a.m[r] = M == -INFINITY ? -INFINITY : M * PA_LN2; a.l[r] = L; }
}

hipError_t launch_merge(int hd, const MergeArgs & a, hipStream_t st) {
    const uint32_t grid = a.nkv * a.rows;
    if (a.n_slots > 16 && a.n_slots <= 64) {                        // many slots: one thread per slot, one wave
        if (hd == 128) hipLaunchKernelGGL((merge_wide_kernel<128, 64>), dim3(grid * 4), dim3(64), 0, st, a);
        else if (hd == 256) hipLaunchKernelGGL((merge_wide_kernel<256, 64>), dim3(grid * 8), dim3(64), 0, st, a);
        else return hipErrorInvalidValue;
        return hipGetLastError();
    }
    if (a.n_slots > 64 && a.n_slots <= 256) {                       // up to 256: four waves
        if (hd == 128) hipLaunchKernelGGL((merge_wide_kernel<128, 256>), dim3(grid * 4), dim3(256), 0, st, a);
        else if (hd == 256) hipLaunchKernelGGL((merge_wide_kernel<256, 256>), dim3(grid * 8), dim3(256), 0, st, a);
        else return hipErrorInvalidValue;
        return hipGetLastError();
    }
    if (a.n_slots <= 16) {                                           // few slots: several rows per workgroup
        if (hd == 128) hipLaunchKernelGGL(merge_rows_kernel<128>, dim3((grid + 7) / 8), dim3(256), 0, st, a);
        else if (hd == 256) hipLaunchKernelGGL(merge_rows_kernel<256>, dim3((grid + 3) / 4), dim3(256), 0, st, a);
        else return hipErrorInvalidValue;
        return hipGetLastError();
    }
    if (hd == 128) hipLaunchKernelGGL((merge_batched_kernel<128>), dim3(grid * 4), dim3(256), 0, st, a);
    else if (hd == 256) hipLaunchKernelGGL((merge_batched_kernel<256>), dim3(grid * 8), dim3(256), 0, st, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace pa_hip
