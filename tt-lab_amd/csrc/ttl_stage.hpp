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

#include <type_traits>

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

// Host side: the C ABI's ttl_stage_input as the kernels take it, and its checks.
inline Input from_abi(const ttl_stage_input *in) {
    Input s;
    s.base = in->base;
    s.add = in->add;
    s.add_w = in->add_weights;
    s.add_k = in->add_count;
    s.norm_w = in->norm_weight;
    s.eps = in->epsilon;
    s.v_out = in->sum_out;
    return s;
}

inline int check(const ttl_stage_input *in, const char *who) {
    TTL_REQUIRE(in && in->base, TTL_ERR_INVALID, "%s: null input", who);
    TTL_REQUIRE(((uintptr_t)in->base & 15) == 0, TTL_ERR_INVALID, "%s: input must be 16-byte aligned", who);
    TTL_REQUIRE(!in->add || (in->add_weights && in->add_count >= 1 && in->add_count <= 4 &&
                             ((uintptr_t)in->add & 15) == 0),
                TTL_ERR_INVALID, "%s: the combine needs 1..4 terms, 16-byte aligned", who);
    TTL_REQUIRE(!in->norm_weight || ((uintptr_t)in->norm_weight & 15) == 0, TTL_ERR_INVALID,
                "%s: norm weights must be 16-byte aligned", who);
    TTL_REQUIRE(!in->sum_out || ((uintptr_t)in->sum_out & 15) == 0, TTL_ERR_INVALID,
                "%s: sum_out must be 16-byte aligned", who);
    return TTL_OK;
}

// Which optional steps a staging runs (a template parameter of the kernels, so
// the staging is straight-line code: no branch between issuing the loads and
// using them, which lets the compiler wait for each load only where it is used).
enum Mode : int { kPlain = 0, kNorm = 1, kAdd = 2, kAddNorm = 3 };
constexpr uint32_t kMaxAdd = 4;  // combine terms a staging holds in registers

inline int mode_of(const Input &in) {
    return (in.norm_w ? kNorm : 0) | (in.add ? kAdd : 0);
}

// Calls f(std::integral_constant<int, MODE>{}) for the staging's mode.
template <class F>
inline void with_mode(const Input &in, F &&f) {
    switch (mode_of(in)) {
    case kPlain:
        f(std::integral_constant<int, kPlain>{});
        break;
    case kNorm:
        f(std::integral_constant<int, kNorm>{});
        break;
    case kAdd:
        f(std::integral_constant<int, kAdd>{});
        break;
    default:
        f(std::integral_constant<int, kAddNorm>{});
        break;
    }
}

// Per-thread registers of a staging in flight: the loads of stage_load() land
// here, so a kernel can issue them before its weight loads and finish the
// staging while those are still in flight.
template <int N, int XB, int NT, int MODE>
struct Pending {
    static_assert(N % 32 == 0 && N / 32 <= XB, "vector does not fit the layout");
    static constexpr int groups = (N / 32) * 8;        // float4 groups of the vector
    static constexpr int per = (XB * 8 + NT - 1) / NT;  // layout groups per thread
    static constexpr bool add = (MODE & kAdd) != 0, norm = (MODE & kNorm) != 0;
    float4 v[per];
    float4 a[per][add ? kMaxAdd : 1];
    float4 w[per];
    float aw_lane;  // combine weight lane % kMaxAdd
};

// Issues every global load of the staging, unconditionally: base, the combine
// terms and their weights, the norm weights.  Threads past the vector's end
// re-read its last group (discarded in stage_finish).
template <int N, int XB, int NT, int MODE>
__device__ __attribute__((always_inline)) inline void stage_load(const Input &in, Pending<N, XB, NT, MODE> &p) {
    using P = Pending<N, XB, NT, MODE>;
    const float4 *b4 = reinterpret_cast<const float4 *>(in.base);
    if constexpr (P::add) {
        // lane r of each wave loads weight r (a vector load, issued here; loads from
        // one uniform address go to the scalar unit, and the compiler sinks those to
        // their uses, each behind a wait of its own); stage_finish reads the lanes
        const uint32_t r = threadIdx.x % kMaxAdd;
        p.aw_lane = in.add_w[r < in.add_k ? r : 0];
    }
#pragma unroll
    for (int j = 0; j < P::per; ++j) {
        const uint32_t i = threadIdx.x + uint32_t(j) * NT;
        const uint32_t c = i < uint32_t(P::groups) ? i : uint32_t(P::groups) - 1;
        p.v[j] = b4[c];
        if constexpr (P::norm) {
            p.w[j] = reinterpret_cast<const float4 *>(in.norm_w)[c];
        }
        if constexpr (P::add) {
#pragma unroll
            for (uint32_t r = 0; r < kMaxAdd; ++r) {
                const uint32_t rr = r < in.add_k ? r : 0;
                p.a[j][r] = reinterpret_cast<const float4 *>(in.add + size_t(rr) * N)[c];
            }
        }
    }
}

// Completes a staging begun by stage_load(): writes blocks [0, XB) of the padded
// layout (blocks >= N/32 are zero) and v_out, then applies the norm.  With the norm,
// every wave takes the same sum of squares (the same order in each), so no wave waits
// on another for the scale, and each thread writes its normalized values to LDS once,
// from registers.  blockDim.x == NT.
template <int N, int XB, int NT, int MODE>
__device__ __attribute__((always_inline)) inline void stage_finish(const Input &in, const Pending<N, XB, NT, MODE> &p,
                                                                   float *xs, float *red) {
#pragma clang fp contract(off)
    using P = Pending<N, XB, NT, MODE>;
    float4 kept[P::norm ? P::per : 1];
#pragma unroll
    for (int j = 0; j < P::per; ++j) {
        const uint32_t i = threadIdx.x + uint32_t(j) * NT;
        if (i >= uint32_t(XB) * 8) {
            continue;
        }
        const bool inside = i < uint32_t(P::groups);
        float4 v = inside ? p.v[j] : make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (P::add) {
            // model.cpp:323-337: out = 0; out += w_r * down_r (rank order); then x + out
            float4 m = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (uint32_t r = 0; r < kMaxAdd; ++r) {
                if (r < in.add_k) {
                    const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p.aw_lane), int(r)));
                    const float4 a = p.a[j][r];
                    m.x = m.x + w * a.x;
                    m.y = m.y + w * a.y;
                    m.z = m.z + w * a.z;
                    m.w = m.w + w * a.w;
                }
            }
            if (inside) {
                v.x = v.x + m.x;
                v.y = v.y + m.y;
                v.z = v.z + m.z;
                v.w = v.w + m.w;
            }
        }
        if (inside) {
            if (in.v_out) {
                reinterpret_cast<float4 *>(in.v_out)[i] = v;
            }
            if constexpr (P::norm) {
                red[i] = v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            }
        }
        if constexpr (P::norm) {
            kept[j] = v;
        } else {
            *reinterpret_cast<float4 *>(xs + (i / 8) * x_stride + (i % 8) * 4) = v;
        }
    }
    __syncthreads();
    if constexpr (P::norm) {
        // tensor.cpp:568-580: scale = 1 / sqrt(mean(v^2) + eps); xs = v * scale * w
        const uint32_t lane = threadIdx.x % 64;
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < (P::groups + 63) / 64; ++k) {
            const uint32_t i = lane + 64u * uint32_t(k);
            if (i < uint32_t(P::groups)) {
                s = s + red[i];
            }
        }
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) {
            s = s + __shfl_xor(s, d);
        }
        const float scale = 1.0f / sqrtf(s / float(N) + in.eps);
#pragma unroll
        for (int j = 0; j < P::per; ++j) {
            const uint32_t i = threadIdx.x + uint32_t(j) * NT;
            if (i >= uint32_t(XB) * 8) {
                continue;
            }
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i < uint32_t(P::groups)) {
                const float4 w = p.w[j];
                v.x = kept[j].x * scale * w.x;
                v.y = kept[j].y * scale * w.y;
                v.z = kept[j].z * scale * w.z;
                v.w = kept[j].w * scale * w.w;
            }
            *reinterpret_cast<float4 *>(xs + (i / 8) * x_stride + (i % 8) * 4) = v;
        }
        __syncthreads();
    }
}

// Both halves at once, for kernels with nothing else to load first.
template <int N, int XB, int NT, int MODE>
__device__ __attribute__((always_inline)) inline void stage(const Input &in, float *xs, float *red) {
    Pending<N, XB, NT, MODE> p;
    stage_load(in, p);
    stage_finish(in, p, xs, red);
}

}  // namespace stage
