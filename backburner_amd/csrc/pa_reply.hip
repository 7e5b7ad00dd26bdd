// pa_reply.hip - the reply side of an attention call on the device: the LSE merge of two partials, the reply format
// (normalised f16 O and lse), and the receiver's co-attention merge of a reply with its own partial (gfx950).
//
// One wave per row, HD / 64 consecutive floats per lane, four rows per 256-thread workgroup. A row's (m, l) is read by
// every lane of its wave before any lane writes it, so the in-place merge needs no synchronisation. Every expression
// rounds as written (no contraction), as the reference's host loops do.
//
// Reference roles:
//   pa_merge_partial_kernel  pa::merge_partial (phone-attn.h:231-239): the server's merge of engine partials
//   pa_normalise_kernel      the ATTN reply (phone-attn.h:651-655): Oh = f16(O / l), lse = m + log l
//   pa_coattn_kernel         the receiver's co-attention slot (phone-attn.h:21: the reply enters its attention as
//                            O_unnorm = O, S = 1, M = lse), merged as pa::merge_partial does, then normalised
#include "pa_attn.h"
#include "pa_common.h"

namespace pa_hip {

template <int HD> struct RowVec {
    static constexpr int N = HD / 64;                           // floats per lane: 2 (hd 128) or 4 (hd 256)
};

template <int N> __device__ __forceinline__ void ld_f(const float * p, float (&v)[N]) {
    if constexpr (N == 2) { const float2 x = *(const float2 *) p; v[0] = x.x; v[1] = x.y; }
    else { const float4 x = *(const float4 *) p; v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w; }
}
template <int N> __device__ __forceinline__ void st_f(float * p, const float (&v)[N]) {
    if constexpr (N == 2) *(float2 *) p = make_float2(v[0], v[1]);
    else *(float4 *) p = make_float4(v[0], v[1], v[2], v[3]);
}
template <int N> __device__ __forceinline__ void ld_h(const uint16_t * p, float (&v)[N]) {
    if constexpr (N == 2) { const pa_h2 x = *(const pa_h2 *) p; v[0] = (float) x[0]; v[1] = (float) x[1]; }
    else { const pa_h4 x = *(const pa_h4 *) p; for (int k = 0; k < 4; k++) v[k] = (float) x[k]; }
}
template <int N> __device__ __forceinline__ void st_h(uint16_t * p, const float (&v)[N]) {
    if constexpr (N == 2) *(pa_h2 *) p = (pa_h2){(_Float16) v[0], (_Float16) v[1]};
    else *(pa_h4 *) p = (pa_h4){(_Float16) v[0], (_Float16) v[1], (_Float16) v[2], (_Float16) v[3]};
}

// fold (O2, m2, l2) into (O, m, l), natural-log units
template <int HD>
__global__ __launch_bounds__(256) void pa_merge_partial_kernel(float * O, float * m, float * l, const float * O2,
                                                               const float * m2, const float * l2, uint64_t rows) {
    #pragma clang fp contract(off)
    constexpr int N = RowVec<HD>::N;
    const uint64_t r = (uint64_t) blockIdx.x * 4 + threadIdx.x / 64;
    const int lane = threadIdx.x % 64;
    if (r >= rows) return;
    const float lb = l2[r];
    if (lb <= 0.0f) return;                                      // l2 <= 0: nothing to add
    const float la = l[r], ma = m[r], mb = m2[r];
    float o[N], o2[N];
    ld_f<N>(O2 + r * HD + N * lane, o2);
    if (la <= 0.0f) {                                            // l <= 0: take the second partial as it is
        st_f<N>(O + r * HD + N * lane, o2);
        if (lane == 0) { m[r] = mb; l[r] = lb; }
        return;
    }
    const float M = fmaxf(ma, mb), wa = expf(ma - M), wb = expf(mb - M);
    ld_f<N>(O + r * HD + N * lane, o);
    #pragma unroll
    for (int k = 0; k < N; k++) o[k] = o[k] * wa + o2[k] * wb;
    st_f<N>(O + r * HD + N * lane, o);
    if (lane == 0) { m[r] = M; l[r] = la * wa + lb * wb; }
}

// Oh = f16(O * (1 / l)) (0 where l <= 0), lse = m + log l (-inf where l <= 0)
template <int HD>
__global__ __launch_bounds__(256) void pa_normalise_kernel(const float * O, const float * m, const float * l, uint64_t rows,
                                                           uint16_t * Oh, float * lse) {
    #pragma clang fp contract(off)
    constexpr int N = RowVec<HD>::N;
    const uint64_t r = (uint64_t) blockIdx.x * 4 + threadIdx.x / 64;
    const int lane = threadIdx.x % 64;
    if (r >= rows) return;
    const float lr = l[r];
    const float inv = lr > 0.0f ? 1.0f / lr : 0.0f;
    float o[N];
    ld_f<N>(O + r * HD + N * lane, o);
    #pragma unroll
    for (int k = 0; k < N; k++) o[k] = pa_f32(o[k] * inv);     // rounded to fp32, then to fp16 (as f2h(O * inv))
    st_h<N>(Oh + r * HD + N * lane, o);
    if (lane == 0) lse[r] = lr > 0.0f ? m[r] + logf(lr) : -INFINITY;
}

// out = the local partial (O_loc, m_loc, l_loc) merged with the reply (Oh, S = 1, M = lse), then normalised;
// lse_out (optional) = the merged m + log l
template <int HD>
__global__ __launch_bounds__(256) void pa_coattn_kernel(const uint16_t * Oh, const float * lse, const float * Oloc,
                                                        const float * mloc, const float * lloc, uint64_t rows, float * out,
                                                        float * lse_out) {
    #pragma clang fp contract(off)
    constexpr int N = RowVec<HD>::N;
    const uint64_t r = (uint64_t) blockIdx.x * 4 + threadIdx.x / 64;
    const int lane = threadIdx.x % 64;
    if (r >= rows) return;
    const float la = lloc[r], ma = mloc[r], mb = lse[r];
    float o[N], o2[N];
    ld_h<N>(Oh + r * HD + N * lane, o2);
    float M, L;
    if (la <= 0.0f) {                                            // no local keys: the reply as it is
        #pragma unroll
        for (int k = 0; k < N; k++) o[k] = o2[k];
        M = mb; L = 1.0f;
    } else {
        M = fmaxf(ma, mb);
        const float wa = expf(ma - M), wb = expf(mb - M);
        ld_f<N>(Oloc + r * HD + N * lane, o);
        #pragma unroll
        for (int k = 0; k < N; k++) o[k] = o[k] * wa + o2[k] * wb;
        L = la * wa + 1.0f * wb;
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    #pragma unroll
    for (int k = 0; k < N; k++) o[k] = o[k] * inv;
    st_f<N>(out + r * HD + N * lane, o);
    if (lse_out && lane == 0) lse_out[r] = L > 0.0f ? M + logf(L) : -INFINITY;
}

hipError_t launch_merge_partial(int hd, float * O, float * m, float * l, const float * O2, const float * m2, const float * l2,
                                uint64_t rows, hipStream_t st) {
    if (rows == 0) return hipSuccess;
    const dim3 grid((unsigned) ((rows + 3) / 4));
    if (hd == 128) hipLaunchKernelGGL(pa_merge_partial_kernel<128>, grid, dim3(256), 0, st, O, m, l, O2, m2, l2, rows);
    else if (hd == 256) hipLaunchKernelGGL(pa_merge_partial_kernel<256>, grid, dim3(256), 0, st, O, m, l, O2, m2, l2, rows);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_normalise(int hd, const float * O, const float * m, const float * l, uint64_t rows, uint16_t * Oh,
                            float * lse, hipStream_t st) {
    if (rows == 0) return hipSuccess;
    const dim3 grid((unsigned) ((rows + 3) / 4));
    if (hd == 128) hipLaunchKernelGGL(pa_normalise_kernel<128>, grid, dim3(256), 0, st, O, m, l, rows, Oh, lse);
    else if (hd == 256) hipLaunchKernelGGL(pa_normalise_kernel<256>, grid, dim3(256), 0, st, O, m, l, rows, Oh, lse);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_coattn(int hd, const uint16_t * Oh, const float * lse, const float * Oloc, const float * mloc,
                         const float * lloc, uint64_t rows, float * out, float * lse_out, hipStream_t st) {
    if (rows == 0) return hipSuccess;
    const dim3 grid((unsigned) ((rows + 3) / 4));
    if (hd == 128) hipLaunchKernelGGL(pa_coattn_kernel<128>, grid, dim3(256), 0, st, Oh, lse, Oloc, mloc, lloc, rows, out, lse_out);
    else if (hd == 256) hipLaunchKernelGGL(pa_coattn_kernel<256>, grid, dim3(256), 0, st, Oh, lse, Oloc, mloc, lloc, rows, out, lse_out);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace pa_hip
