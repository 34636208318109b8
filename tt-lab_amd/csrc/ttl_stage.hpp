// Staging of a matvec's input vector into LDS, with the elementwise steps that
// precede a matvec in GptOssModel::forward fused in:
//
//   v = base                                   (plain input)
//   v = base + sum_r w_r * add_r               (the MoE combine, model.cpp:323-337, 592-594)
//   xs = rms_norm(v) * weight                  (tensor.cpp:568-580), optional
//
// Every workgroup of every kernel computes the same v and the same norm: the sum
// of squares is taken in one fixed order (per 4-element group, then a fixed
// 64-lane reduction) whatever the workgroup size, so all consumers of a
// normalized vector see identical values.  The reference's sequential sums round
// differently (within the tolerance of the layer outputs).
#pragma once

#include "ttl_internal.hpp"

namespace stage {

constexpr int x_stride = 36;  // padded LDS floats per 32-value block (bank-conflict-free b128 reads)

struct Input {
    const float *base;      // f32 [n], 16-byte aligned
    const float *add;       // f32 [k][n] or null
    const float *add_w;     // f32 [k] (combine weights) or null
    uint32_t add_k;
    const float *norm_w;    // RMSNorm weights f32 [n] or null (no norm)
    float eps;
    float *v_out;           // if non-null, this workgroup writes v (before the norm) here
};

// LDS floats `red` must hold for a vector of x_blocks blocks.
__host__ __device__ constexpr int red_floats(int x_blocks) {
    return x_blocks * 8 + 1;
}

// Writes blocks [0, x_blocks) of the padded layout; blocks >= n/32 are zero.
// blockDim.x must be a multiple of 64.
__device__ inline void stage(const Input &in, uint32_t n, uint32_t x_blocks, float *xs, float *red) {
#pragma clang fp contract(off)
    const uint32_t blocks = n / 32, groups = blocks * 8;
    const float4 *b4 = reinterpret_cast<const float4 *>(in.base);
    for (uint32_t i = threadIdx.x; i < x_blocks * 8; i += blockDim.x) {
        const uint32_t block = i / 8, part = i % 8;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (block < blocks) {
            v = b4[i];
            if (in.add) {
                float4 m = make_float4(0.f, 0.f, 0.f, 0.f);
                for (uint32_t r = 0; r < in.add_k; ++r) {
                    const float w = in.add_w[r];
                    const float4 a = reinterpret_cast<const float4 *>(in.add + size_t(r) * n)[i];
                    m.x = m.x + w * a.x;
                    m.y = m.y + w * a.y;
                    m.z = m.z + w * a.z;
                    m.w = m.w + w * a.w;
                }
                v.x = v.x + m.x;
                v.y = v.y + m.y;
                v.z = v.z + m.z;
                v.w = v.w + m.w;
            }
            if (in.v_out) {
                reinterpret_cast<float4 *>(in.v_out)[i] = v;
            }
            if (in.norm_w) {
                red[i] = v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            }
        }
        *reinterpret_cast<float4 *>(xs + block * x_stride + part * 4) = v;
    }
    __syncthreads();
    if (!in.norm_w) {
        return;
    }
    if (threadIdx.x < 64) {
        float s = 0.0f;
        for (uint32_t i = threadIdx.x; i < groups; i += 64) {
            s = s + red[i];
        }
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) {
            s = s + __shfl_xor(s, d);
        }
        if (threadIdx.x == 0) {
            red[x_blocks * 8] = 1.0f / sqrtf(s / float(n) + in.eps);
        }
    }
    __syncthreads();
    const float scale = red[x_blocks * 8];
    const float4 *w4 = reinterpret_cast<const float4 *>(in.norm_w);
    for (uint32_t i = threadIdx.x; i < groups; i += blockDim.x) {
        const uint32_t block = i / 8, part = i % 8;
        float4 *p = reinterpret_cast<float4 *>(xs + block * x_stride + part * 4);
        float4 v = *p;
        const float4 w = w4[i];
        v.x = v.x * scale * w.x;
        v.y = v.y * scale * w.y;
        v.z = v.z * scale * w.z;
        v.w = v.w * scale * w.w;
        *p = v;
    }
    __syncthreads();
}

}  // namespace stage
