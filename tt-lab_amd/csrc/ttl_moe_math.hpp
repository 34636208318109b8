// Scalar arithmetic of the MoE layer shared by the decode and prefill kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace moe_math {

// std::max / std::min as the reference's libstdc++ defines them.
__device__ inline float std_max(float a, float b) {
    return (a < b) ? b : a;
}
__device__ inline float std_min(float a, float b) {
    return (b < a) ? b : a;
}

// model.cpp:328-332: x = std::min(gate, 7), y = std::clamp(up, -7, 7),
// h = (x / (1 + exp(-1.702 x))) * (y + 1), no multiply-add contraction.
__device__ inline float clamped_swiglu(float gate, float up) {
#pragma clang fp contract(off)
    const float x = std_min(gate, 7.0f);
    const float y = (up < -7.0f) ? -7.0f : ((7.0f < up) ? 7.0f : up);
    return (x / (1.0f + expf(-1.702f * x))) * (y + 1.0f);
}

// The same clamps and NaN behaviour with the hardware exponential and reciprocal
// (a few ulp): for the scaled prefill path, whose hidden is rounded to E4M3 (3
// fraction bits) right after, so the difference almost never reaches a stored bit.
__device__ inline float clamped_swiglu_fast(float gate, float up) {
    const float x = std_min(gate, 7.0f);
    const float y = (up < -7.0f) ? -7.0f : ((7.0f < up) ? 7.0f : up);
    return x * __builtin_amdgcn_rcpf(1.0f + __expf(-1.702f * x)) * (y + 1.0f);
}

}  // namespace moe_math
