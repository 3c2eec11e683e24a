// Elementwise consumers of fp32 operator outputs: the SwiGLU gate silu(g) * u and the
// residual add h + y, each rounded once to the output type.
//
// Role of consume_silu_mul / consume_add (csrc/v3g/bind.cu:96-149), which read the
// reference's persistent fp32 workspace and zero it for the next call. Outputs here are
// ordinary tensors, so the inputs are only read. The same arithmetic is also fused into
// the operator's own output store (trk_forward_epilogue), which is the faster path; these
// serve callers that hold fp32 outputs from elsewhere.
//
// HBM-bound: 4 elements per thread, the fp32 inputs read with 16-byte loads when they are
// 16-byte aligned, in a grid-stride loop over at most 8 workgroups per CU.
#include <algorithm>

#include "trk_internal.h"
#include "trk_types.h"

namespace trk {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxGroups = 256 * 8;

template <int DT, int VEC>
__global__ void __launch_bounds__(kThreads)
    silu_mul_kernel(const float *__restrict__ g, const float *__restrict__ u,
                    typename Elem<DT>::T *__restrict__ out, size_t n) {
    using E = Elem<DT>;
    const size_t stride = size_t(gridDim.x) * kThreads * VEC;
    for (size_t i = (size_t(blockIdx.x) * kThreads + threadIdx.x) * VEC; i < n; i += stride) {
        if constexpr (VEC == 4) {
            if (i + 4 <= n) {
                const float4 a = *reinterpret_cast<const float4 *>(g + i);
                const float4 b = *reinterpret_cast<const float4 *>(u + i);
                out[i] = E::from_f32(silu_f32(a.x) * b.x);
                out[i + 1] = E::from_f32(silu_f32(a.y) * b.y);
                out[i + 2] = E::from_f32(silu_f32(a.z) * b.z);
                out[i + 3] = E::from_f32(silu_f32(a.w) * b.w);
                continue;
            }
        }
        for (size_t j = i; j < i + VEC && j < n; ++j) out[j] = E::from_f32(silu_f32(g[j]) * u[j]);
    }
}

template <int DT, int VEC>
__global__ void __launch_bounds__(kThreads)
    add_kernel(const typename Elem<DT>::T *h, const float *__restrict__ y,
               typename Elem<DT>::T *out, size_t n) {  // out may equal h
    using E = Elem<DT>;
    const size_t stride = size_t(gridDim.x) * kThreads * VEC;
    for (size_t i = (size_t(blockIdx.x) * kThreads + threadIdx.x) * VEC; i < n; i += stride) {
        if constexpr (VEC == 4) {
            if (i + 4 <= n) {
                const float4 b = *reinterpret_cast<const float4 *>(y + i);
                const float a0 = E::to_f32(h[i]), a1 = E::to_f32(h[i + 1]);
                const float a2 = E::to_f32(h[i + 2]), a3 = E::to_f32(h[i + 3]);
                out[i] = E::from_f32(a0 + b.x);
                out[i + 1] = E::from_f32(a1 + b.y);
                out[i + 2] = E::from_f32(a2 + b.z);
                out[i + 3] = E::from_f32(a3 + b.w);
                continue;
            }
        }
        for (size_t j = i; j < i + VEC && j < n; ++j) out[j] = E::from_f32(E::to_f32(h[j]) + y[j]);
    }
}

unsigned groups_for(size_t n, int vec) {
    const size_t per = size_t(kThreads) * vec;
    return unsigned(std::min<size_t>((n + per - 1) / per, kMaxGroups));
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

int launch_silu_mul(const float *g, const float *u, void *out, int out_dtype, size_t n,
                    hipStream_t stream) {
    if (n == 0) return TRK_OK;
    const bool vec = aligned16(g) && aligned16(u);
    switch (out_dtype) {
#define TRK_SILU_MUL(DT)                                                                      \
    case DT: {                                                                                \
        using T = Elem<DT>::T;                                                                \
        if (vec)                                                                              \
            hipLaunchKernelGGL((silu_mul_kernel<DT, 4>), dim3(groups_for(n, 4)), dim3(kThreads), \
                               0, stream, g, u, static_cast<T *>(out), n);                    \
        else                                                                                  \
            hipLaunchKernelGGL((silu_mul_kernel<DT, 1>), dim3(groups_for(n, 1)), dim3(kThreads), \
                               0, stream, g, u, static_cast<T *>(out), n);                    \
        break;                                                                                \
    }
        TRK_SILU_MUL(TRK_DTYPE_F16)
        TRK_SILU_MUL(TRK_DTYPE_BF16)
        TRK_SILU_MUL(TRK_DTYPE_F32)
#undef TRK_SILU_MUL
        default:
            return set_error(TRK_ERR_INVALID, "trk_consume_silu_mul: unknown dtype %d", out_dtype);
    }
    return check_hip(hipGetLastError(), "trk_consume_silu_mul: launch");
}

int launch_add(const void *h, const float *y, void *out, int dtype, size_t n, hipStream_t stream) {
    if (n == 0) return TRK_OK;
    const bool vec = aligned16(y);
    switch (dtype) {
#define TRK_ADD(DT)                                                                            \
    case DT: {                                                                                 \
        using T = Elem<DT>::T;                                                                 \
        if (vec)                                                                               \
            hipLaunchKernelGGL((add_kernel<DT, 4>), dim3(groups_for(n, 4)), dim3(kThreads), 0,  \
                               stream, static_cast<const T *>(h), y, static_cast<T *>(out), n); \
        else                                                                                   \
            hipLaunchKernelGGL((add_kernel<DT, 1>), dim3(groups_for(n, 1)), dim3(kThreads), 0,  \
                               stream, static_cast<const T *>(h), y, static_cast<T *>(out), n); \
        break;                                                                                 \
    }
        TRK_ADD(TRK_DTYPE_F16)
        TRK_ADD(TRK_DTYPE_BF16)
        TRK_ADD(TRK_DTYPE_F32)
#undef TRK_ADD
        default:
            return set_error(TRK_ERR_INVALID, "trk_consume_add: unknown dtype %d", dtype);
    }
    return check_hip(hipGetLastError(), "trk_consume_add: launch");
}

}  // namespace trk
