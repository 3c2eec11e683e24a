// Element types of libtrk kernels: storage type and fp32 conversions per trk_dtype.
#pragma once

#include <hip/hip_runtime.h>

#include "trk.h"
#include "trk_internal.h"

namespace trk {

template <int DT>
struct Elem;

template <>
struct Elem<TRK_DTYPE_F16> {
    using T = _Float16;
    __device__ static float to_f32(T v) { return static_cast<float>(v); }
    __device__ static T from_f32(float v) { return static_cast<T>(v); }  // round to nearest even
};

template <>
struct Elem<TRK_DTYPE_BF16> {
    using T = __bf16;
    __device__ static float to_f32(T v) { return static_cast<float>(v); }
    __device__ static T from_f32(float v) { return static_cast<T>(v); }  // round to nearest even
};

template <>
struct Elem<TRK_DTYPE_F32> {
    using T = float;
    __device__ static float to_f32(T v) { return v; }
    __device__ static T from_f32(float v) { return v; }
};

// silu(a) = a * sigmoid(a) = a / (1 + e^-a), fp32. For large negative a, e^-a overflows to
// +inf and the quotient is -0; for large positive a it tends to a.
__device__ inline float silu_f32(float a) { return a / (1.0f + expf(-a)); }

// Output epilogues (struct Epi). epi_aux reads the aux input of element o (the plan's type, or
// fp32 with kAuxF32; 0 for the kinds that read none); epi_put stores element o of v (fp32)
// combined with that input: y holds the plan's element type, or fp32 for TRK_EPI_F32.
template <int DT>
__device__ inline float epi_aux(const void *aux, int mode, size_t o) {
    using E = Elem<DT>;
    const int kind = mode & kEpiKindMask;
    if (kind != TRK_EPI_ADD && kind != TRK_EPI_SILU_MUL) return 0.0f;
    return (mode & kAuxF32) ? static_cast<const float *>(aux)[o]
                            : E::to_f32(static_cast<const typename E::T *>(aux)[o]);
}

template <int DT>
__device__ inline void epi_put(void *y, int mode, size_t o, float v, float a) {
    using E = Elem<DT>;
    switch (mode & kEpiKindMask) {
        case TRK_EPI_F32: static_cast<float *>(y)[o] = v; return;
        case TRK_EPI_ADD: v = a + v; break;
        case TRK_EPI_SILU_MUL: v = silu_f32(a) * v; break;
        default: break;
    }
    static_cast<typename E::T *>(y)[o] = E::from_f32(v);
}

}  // namespace trk
