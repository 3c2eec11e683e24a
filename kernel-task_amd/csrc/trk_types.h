// Element types of libtrk kernels: storage type and fp32 conversions per trk_dtype.
#pragma once

#include <hip/hip_runtime.h>

#include "trk.h"

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

}  // namespace trk
