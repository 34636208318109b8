// Attention with sinks for one decode token (GptOssModel::attention_from_cache,
// model.cpp:255-290), split over chunks of 64 cached positions.
//
//  partial: workgroup (chunk c, kv head h) scores the 8 query heads that share h
//           (GQA, head/8 = h) against positions of chunk c, and keeps per head the
//           chunk max m_c, sum l_c = sum exp(s - m_c) and o_c = sum exp(s - m_c) v.
//  combine: per query head, M = max(sink, max_c m_c),
//           den = exp(sink - M) + sum_c l_c exp(m_c - M),
//           out = sum_c o_c exp(m_c - M) / den -- the reference's softmax with the
//           sink in the max and the denominator only, regrouped by chunk.
// Even layers see the last 128 positions (the sliding window), odd layers all
// (model.cpp:260).  The position is read from device memory, so one captured
// launch serves every decode step; chunks past the current length do nothing.
#include "ttl_internal.hpp"

#include <cmath>

namespace {

constexpr int kHead = 64, kQHeads = 64, kKvHeads = 8, kGroup = kQHeads / kKvHeads;
constexpr int kChunk = 64, kWindow = 128;
constexpr int kThreads = 256;

struct Span {
    uint32_t first, count;
};

__device__ inline Span span_of(uint32_t pos, uint32_t layer_index) {
    const uint32_t first = (layer_index % 2 == 0 && pos + 1 > uint32_t(kWindow)) ? pos + 1 - kWindow : 0;
    return {first, pos + 1 - first};
}

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        v = fmaxf(v, __shfl_xor(v, d));
    }
    return v;
}

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        v += __shfl_xor(v, d);
    }
    return v;
}

__global__ __launch_bounds__(kThreads) void attn_partial_kernel(const float *__restrict__ q,
                                                                const float *__restrict__ k_cache,
                                                                const float *__restrict__ v_cache,
                                                                const int32_t *__restrict__ position,
                                                                uint32_t capacity, uint32_t layer_index,
                                                                uint32_t max_chunks, float *__restrict__ o_part,
                                                                float2 *__restrict__ ml_part) {
    __shared__ __attribute__((aligned(16))) float qs[kGroup][kHead];
    __shared__ float e[kGroup][kChunk];
    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y, t = threadIdx.x;
    const uint32_t pos = uint32_t(*position);
    if (pos >= capacity) {
        return;
    }
    const Span sp = span_of(pos, layer_index);
    const uint32_t start = sp.first + chunk * kChunk;
    if (chunk * kChunk >= sp.count) {
        return;
    }
    const uint32_t n = min(uint32_t(kChunk), sp.count - chunk * kChunk);
    for (uint32_t i = t; i < kGroup * kHead; i += kThreads) {
        qs[i / kHead][i % kHead] = q[(kvh * kGroup) * kHead + i];
    }
    __syncthreads();

    // scores: thread (p = t % 64, heads 2*(t/64), 2*(t/64)+1)
    {
        const uint32_t p = t % kChunk, g0 = 2 * (t / kChunk);
        float s0 = -INFINITY, s1 = -INFINITY;
        if (p < n) {
            const float4 *k4 = reinterpret_cast<const float4 *>(k_cache + (size_t(start + p) * kKvHeads + kvh) * kHead);
            float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
            for (int d = 0; d < kHead / 4; ++d) {
                const float4 kv = k4[d];
                const float4 qa = *reinterpret_cast<const float4 *>(&qs[g0][4 * d]);
                const float4 qb = *reinterpret_cast<const float4 *>(&qs[g0 + 1][4 * d]);
                a0 = fmaf(qa.x, kv.x, a0);
                a0 = fmaf(qa.y, kv.y, a0);
                a0 = fmaf(qa.z, kv.z, a0);
                a0 = fmaf(qa.w, kv.w, a0);
                a1 = fmaf(qb.x, kv.x, a1);
                a1 = fmaf(qb.y, kv.y, a1);
                a1 = fmaf(qb.z, kv.z, a1);
                a1 = fmaf(qb.w, kv.w, a1);
            }
            s0 = a0 * 0.125f;  // 1/sqrt(64), exact
            s1 = a1 * 0.125f;
        }
        e[g0][p] = s0;
        e[g0 + 1][p] = s1;
    }
    __syncthreads();
    // per head: chunk max and exp sums (wave w handles heads 2w, 2w+1; lane = position)
    {
        const uint32_t w = t / 64, lane = t % 64;
        for (uint32_t g = 2 * w; g < 2 * w + 2; ++g) {
            const float s = e[g][lane];
            const float m = wave_max(s);
            const float x = lane < n ? expf(s - m) : 0.0f;
            const float l = wave_sum(x);
            e[g][lane] = x;
            if (lane == 0) {
                ml_part[(size_t(kvh * kGroup + g)) * max_chunks + chunk] = make_float2(m, l);
            }
        }
    }
    __syncthreads();
    // o_c[g][d] = sum_p e[g][p] v[p][d]: thread (g = t/32, dims 2*(t%32), 2*(t%32)+1)
    {
        const uint32_t g = t / 32, d = 2 * (t % 32);
        float o0 = 0.0f, o1 = 0.0f;
        for (uint32_t p = 0; p < n; ++p) {
            const float2 v = *reinterpret_cast<const float2 *>(v_cache + (size_t(start + p) * kKvHeads + kvh) * kHead + d);
            const float x = e[g][p];
            o0 = fmaf(x, v.x, o0);
            o1 = fmaf(x, v.y, o1);
        }
        float *dst = o_part + ((size_t(kvh * kGroup + g)) * max_chunks + chunk) * kHead + d;
        dst[0] = o0;
        dst[1] = o1;
    }
}

__global__ __launch_bounds__(kHead) void attn_combine_kernel(const float *__restrict__ o_part,
                                                             const float2 *__restrict__ ml_part,
                                                             const float *__restrict__ sinks,
                                                             const int32_t *__restrict__ position,
                                                             uint32_t capacity, uint32_t layer_index,
                                                             uint32_t max_chunks, float *__restrict__ out) {
    const uint32_t head = blockIdx.x, d = threadIdx.x;
    const uint32_t pos = uint32_t(*position);
    if (pos >= capacity) {
        return;
    }
    const Span sp = span_of(pos, layer_index);
    const uint32_t chunks = (sp.count + kChunk - 1) / kChunk;
    const float sink = sinks[head];
    float m = sink;
    for (uint32_t c = 0; c < chunks; ++c) {
        m = fmaxf(m, ml_part[size_t(head) * max_chunks + c].x);
    }
    float den = expf(sink - m), acc = 0.0f;
    for (uint32_t c = 0; c < chunks; ++c) {
        const float2 ml = ml_part[size_t(head) * max_chunks + c];
        const float f = expf(ml.x - m);
        den += ml.y * f;
        acc = fmaf(o_part[(size_t(head) * max_chunks + c) * kHead + d], f, acc);
    }
    out[head * kHead + d] = acc / den;
}

}  // namespace

namespace ttl {
// Workspace floats needed by ttl_attention_decode for a given capacity.
size_t attention_partials_floats(uint32_t capacity) {
    const size_t chunks = (capacity + kChunk - 1) / kChunk;
    return size_t(kQHeads) * chunks * (kHead + 2);
}
}  // namespace ttl

extern "C" {

size_t ttl_attention_workspace_bytes(uint32_t capacity) {
    return ttl::attention_partials_floats(capacity) * sizeof(float);
}

int ttl_attention_decode(ttl_ctx *ctx, const float *q_dev, const float *k_cache_dev, const float *v_cache_dev,
                         const float *sinks_dev, const int32_t *position_dev, uint32_t capacity, uint32_t layer_index,
                         float *workspace_dev, float *out_dev) {
    TTL_REQUIRE(ctx && q_dev && k_cache_dev && v_cache_dev && sinks_dev && position_dev && workspace_dev && out_dev,
                TTL_ERR_INVALID, "ttl_attention_decode: null argument");
    TTL_REQUIRE(capacity > 0, TTL_ERR_SHAPE, "ttl_attention_decode: capacity must be positive");
    TTL_REQUIRE(((uintptr_t)q_dev & 15) == 0 && ((uintptr_t)k_cache_dev & 15) == 0 && ((uintptr_t)v_cache_dev & 7) == 0,
                TTL_ERR_INVALID, "ttl_attention_decode: q/k must be 16-byte and v 8-byte aligned");
    const uint32_t max_chunks = (capacity + kChunk - 1) / kChunk;
    // even layers never need more than the window's chunks (plus one for misalignment)
    const uint32_t launch_chunks = layer_index % 2 == 0 ? min(max_chunks, uint32_t(kWindow / kChunk + 1)) : max_chunks;
    float *o_part = workspace_dev;
    float2 *ml_part = reinterpret_cast<float2 *>(workspace_dev + size_t(kQHeads) * max_chunks * kHead);
    attn_partial_kernel<<<dim3(launch_chunks, kKvHeads), kThreads, 0, ctx->stream>>>(
        q_dev, k_cache_dev, v_cache_dev, position_dev, capacity, layer_index, max_chunks, o_part, ml_part);
    TTL_LAUNCHED("attn_partial_kernel");
    attn_combine_kernel<<<kQHeads, kHead, 0, ctx->stream>>>(o_part, ml_part, sinks_dev, position_dev, capacity,
                                                            layer_index, max_chunks, out_dev);
    TTL_LAUNCHED("attn_combine_kernel");
    return TTL_OK;
}

}  // extern "C"
