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
// Even layers see the last 128 positions (the sliding window, one launch of
// attn_window_kernel), odd layers all (model.cpp:260).  The position is read from device memory, so one captured
// launch serves every decode step; chunks past the current length do nothing.
#include "ttl_internal.hpp"
#include "ttl_mfma.hpp"

#include <cmath>
#include <mutex>

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

// LDS row stride of the staged K/V chunk: 68 floats, so the 64 lanes of a score
// pass (one position each) read rows that start in different banks.
constexpr int kRowStride = kHead + 4;

__global__ __launch_bounds__(kThreads) void attn_partial_kernel(const float *__restrict__ q,
                                                                const float *__restrict__ k_cache,
                                                                const float *__restrict__ v_cache,
                                                                const int32_t *__restrict__ position,
                                                                uint32_t capacity, uint32_t layer_index,
                                                                uint32_t max_chunks, float *__restrict__ o_part,
                                                                float2 *__restrict__ ml_part) {
    __shared__ __attribute__((aligned(16))) float ks[kChunk * kRowStride];
    __shared__ __attribute__((aligned(16))) float vs[kChunk * kRowStride];
    // every thread stores its query float4 (t % 128) in a slot of its own, so the store
    // needs no branch (under one, the compiler places the K/V loads after it, and the
    // store waits for q alone); the scores read slots 0..127
    __shared__ float4 qs[kThreads];
    __shared__ float e[kGroup][kChunk];
    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y, t = threadIdx.x;
    // Full-context layers only (their span starts at position 0), so the chunk's rows do
    // not depend on the position: the 8 query heads (every thread loads one of their 128
    // float4), the chunk's 64 K and V rows of head kvh (16 float4 per row; rows past
    // the capacity re-read the last) and the position are requested together, one
    // round trip.  Rows past the span's end are read but never used: their scores are
    // masked and the weighted sum stops at the span's end.
    // No early exit (the compiler would sink the loads below it): a workgroup past the
    // span, or of a position past the capacity, computes with a valid count and stores
    // nothing.
    const float4 qv = reinterpret_cast<const float4 *>(q + size_t(kvh) * kGroup * kHead)[t % (kGroup * kHead / 4)];
    constexpr int kPer = kChunk * (kHead / 4) / kThreads;  // 4 float4 of K and of V per thread
    float4 kr[kPer], vr[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const uint32_t f = t + uint32_t(k) * kThreads, p = f / (kHead / 4), d4 = f % (kHead / 4);
        const size_t row = (size_t(min(chunk * kChunk + p, capacity - 1)) * kKvHeads + kvh) * kHead;
        kr[k] = reinterpret_cast<const float4 *>(k_cache + row)[d4];
        vr[k] = reinterpret_cast<const float4 *>(v_cache + row)[d4];
    }
    const uint32_t pos = uint32_t(*position);
    const Span sp = span_of(pos < capacity ? pos : 0u, layer_index);
    const bool live = pos < capacity && chunk * kChunk < sp.count;
    const uint32_t c0 = live ? chunk * kChunk : 0u;
    const uint32_t n = min(uint32_t(kChunk), sp.count - c0);
    qs[t] = qv;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const uint32_t f = t + uint32_t(k) * kThreads, p = f / (kHead / 4), d4 = f % (kHead / 4);
        *reinterpret_cast<float4 *>(ks + p * kRowStride + 4 * d4) = kr[k];
        *reinterpret_cast<float4 *>(vs + p * kRowStride + 4 * d4) = vr[k];
    }
    __syncthreads();

    // scores: thread (p = t % 64, heads 2*(t/64), 2*(t/64)+1)
    {
        const uint32_t p = t % kChunk, g0 = 2 * (t / kChunk);
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int d = 0; d < kHead / 4; ++d) {
            const float4 kv = *reinterpret_cast<const float4 *>(ks + p * kRowStride + 4 * d);
            const float4 qa = qs[g0 * (kHead / 4) + d];
            const float4 qb = qs[(g0 + 1) * (kHead / 4) + d];
            a0 = fmaf(qa.x, kv.x, a0);
            a0 = fmaf(qa.y, kv.y, a0);
            a0 = fmaf(qa.z, kv.z, a0);
            a0 = fmaf(qa.w, kv.w, a0);
            a1 = fmaf(qb.x, kv.x, a1);
            a1 = fmaf(qb.y, kv.y, a1);
            a1 = fmaf(qb.z, kv.z, a1);
            a1 = fmaf(qb.w, kv.w, a1);
        }
        e[g0][p] = p < n ? a0 * 0.125f : -INFINITY;  // 1/sqrt(64), exact
        e[g0 + 1][p] = p < n ? a1 * 0.125f : -INFINITY;
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
            if (lane == 0 && live) {
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
            const float2 v = *reinterpret_cast<const float2 *>(vs + p * kRowStride + d);
            const float x = e[g][p];
            o0 = fmaf(x, v.x, o0);
            o1 = fmaf(x, v.y, o1);
        }
        if (live) {
            float *dst = o_part + ((size_t(kvh * kGroup + g)) * max_chunks + chunk) * kHead + d;
            dst[0] = o0;
            dst[1] = o1;
        }
    }
}

// One workgroup per query head, one thread per dimension.  The chunk statistics
// are read once (a thread per chunk), the rescale factors shared through LDS.
constexpr int kMaxCombineChunks = 256;  // capacity up to 16384 positions

__global__ __launch_bounds__(kHead) void attn_combine_kernel(const float *__restrict__ o_part,
                                                             const float2 *__restrict__ ml_part,
                                                             const float *__restrict__ sinks,
                                                             const int32_t *__restrict__ position,
                                                             uint32_t capacity, uint32_t layer_index,
                                                             uint32_t max_chunks, float *__restrict__ out) {
    __shared__ float fs[kMaxCombineChunks];
    const uint32_t head = blockIdx.x, d = threadIdx.x;
    // The statistics and the first kEarly chunks' outputs are requested before the
    // position (the chunk count) is known: every address below max_chunks is inside
    // the partials, and chunks past the count are left out below by selection (their
    // stale contents never enter an arithmetic operation).
    constexpr int kPer = kMaxCombineChunks / kHead;
    float2 ml[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        ml[k] = ml_part[size_t(head) * max_chunks + min(d + uint32_t(k) * kHead, max_chunks - 1)];
    }
    constexpr int kEarly = 32;
    const float *op = o_part + size_t(head) * max_chunks * kHead + d;
    float early[kEarly];
#pragma unroll
    for (int c = 0; c < kEarly; ++c) {
        early[c] = op[size_t(min(uint32_t(c), max_chunks - 1)) * kHead];
    }
    __builtin_amdgcn_sched_barrier(0);  // all of them issued before the position is read
    const float sink = sinks[head];
    // no early exit (the compiler would sink the loads above below it): a position
    // past the capacity combines position 0's span and stores nothing
    const uint32_t pos = uint32_t(*position);
    const Span sp = span_of(pos < capacity ? pos : 0u, layer_index);
    const uint32_t chunks = (sp.count + kChunk - 1) / kChunk;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        if (d + uint32_t(k) * kHead >= chunks) {
            ml[k] = make_float2(-INFINITY, 0.0f);
        }
    }
    float m = sink;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        m = fmaxf(m, ml[k].x);
    }
    m = wave_max(m);
    float den = 0.0f;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const uint32_t c = d + uint32_t(k) * kHead;
        const float f = c < chunks ? expf(ml[k].x - m) : 0.0f;
        den += ml[k].y * f;
        fs[c] = f;
    }
    den = wave_sum(den) + expf(sink - m);
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < kEarly; ++c) {
        if (uint32_t(c) < chunks) {
            acc = fmaf(early[c], fs[c], acc);
        }
    }
#pragma unroll 8
    for (uint32_t c = kEarly; c < chunks; ++c) {
        acc = fmaf(op[size_t(c) * kHead], fs[c], acc);
    }
    if (pos < capacity) {
        out[head * kHead + d] = acc / den;
    }
}

// Sliding-window layers in one launch: workgroup = query head; the window (at most
// 128 positions of its kv head) sits in LDS, and the softmax with the sink is done
// in place -- no partials and no second kernel.  512 threads: each score is four
// 16-dimension partial dots added in LDS, each output dimension eight 16-position
// partial sums, so no thread's dependent chain is longer than 16 multiply-adds
// (5.54 -> 5.03 us per launch against 256 threads with 64- and 32-long chains).
constexpr int kWinThreads = 512;

__global__ __launch_bounds__(kWinThreads) void attn_window_kernel(const float *__restrict__ q,
                                                                  const float *__restrict__ k_cache,
                                                                  const float *__restrict__ v_cache,
                                                                  const float *__restrict__ sinks,
                                                                  const int32_t *__restrict__ position,
                                                                  uint32_t capacity, uint32_t layer_index,
                                                                  float *__restrict__ out) {
    __shared__ __attribute__((aligned(16))) float ks[kWindow * kRowStride];
    __shared__ __attribute__((aligned(16))) float vs[kWindow * kRowStride];
    __shared__ float4 qs[kWinThreads];  // thread t's copy of q float4 t % 16 (no branch)
    __shared__ float e[kWindow];
    __shared__ float sq[4][kWindow];
    __shared__ float stat[4];
    __shared__ float part[kWinThreads / kHead][kHead];
    // Workgroups are dealt to the 8 XCDs in turn (workgroup b to XCD b % 8), each XCD with
    // its own L2: workgroup b takes query head 8 (b % 8) + b / 8, so the 8 heads that read
    // one kv head's window run on one XCD and share its L2 (with head = b the window was
    // fetched once per XCD, 7.6 times its bytes).
    const uint32_t head = (blockIdx.x % kKvHeads) * kGroup + blockIdx.x / kKvHeads, kvh = head / kGroup;
    const uint32_t t = threadIdx.x;
    // q and the sink first (one of q's 16 float4 per thread), then the position, then the
    // window's K and V rows (positions past n re-read the last): two round trips
    const float4 qv = reinterpret_cast<const float4 *>(q + size_t(head) * kHead)[t % (kHead / 4)];
    const float sink = sinks[head];
    // no early exit (the compiler would sink the loads above below it): a position
    // past the capacity attends over position 0 and stores nothing
    const uint32_t pos = uint32_t(*position);
    const Span sp = span_of(pos < capacity ? pos : 0u, layer_index);
    const uint32_t n = sp.count;  // 1..128

    constexpr int kPer = kWindow * (kHead / 4) / kWinThreads;  // 4 float4 of K and of V per thread
    static_assert(kPer == 4, "the window of 128 positions over 512 threads");
    float4 kr[kPer], vr[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const uint32_t f = t + uint32_t(k) * kWinThreads, p = f / (kHead / 4), d4 = f % (kHead / 4);
        const size_t row = (size_t(sp.first + (p < n ? p : n - 1)) * kKvHeads + kvh) * kHead;
        kr[k] = reinterpret_cast<const float4 *>(k_cache + row)[d4];
        vr[k] = reinterpret_cast<const float4 *>(v_cache + row)[d4];
    }
    qs[t] = qv;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const uint32_t f = t + uint32_t(k) * kWinThreads, p = f / (kHead / 4), d4 = f % (kHead / 4);
        *reinterpret_cast<float4 *>(ks + p * kRowStride + 4 * d4) = kr[k];
        *reinterpret_cast<float4 *>(vs + p * kRowStride + 4 * d4) = vr[k];
    }
    __syncthreads();

    // scores: thread (position t % 128, dims 16 (t / 128) .. + 15), the quarters added in LDS
    const uint32_t w = t / 64, lane = t % 64;
    {
        const uint32_t p = t % kWindow, qd = t / kWindow;
        float a = 0.0f;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const float4 kv = *reinterpret_cast<const float4 *>(ks + p * kRowStride + 16 * qd + 4 * d);
            const float4 qq = qs[4 * qd + d];
            a = fmaf(qq.x, kv.x, a);
            a = fmaf(qq.y, kv.y, a);
            a = fmaf(qq.z, kv.z, a);
            a = fmaf(qq.w, kv.w, a);
        }
        sq[qd][p] = a;
    }
    __syncthreads();
    if (t < uint32_t(kWindow)) {
        const float a = ((sq[0][t] + sq[1][t]) + sq[2][t]) + sq[3][t];
        const float s = t < n ? a * 0.125f : -INFINITY;  // 1/sqrt(64), exact
        e[t] = s;
        const float m = wave_max(s);
        if (lane == 0) {
            stat[w] = m;
        }
    }
    __syncthreads();
    // model.cpp:270-281: the sink enters the max and the denominator only
    const float m = fmaxf(sink, fmaxf(stat[0], stat[1]));
    if (t < uint32_t(kWindow)) {
        const float x = t < n ? expf(e[t] - m) : 0.0f;
        e[t] = x;
        const float l = wave_sum(x);
        if (lane == 0) {
            stat[2 + w] = l;
        }
    }
    __syncthreads();
    const float den = expf(sink - m) + (stat[2] + stat[3]);
    // o[d] = sum_p e[p] v[p][d]: thread (eighth g = t / 64 of the positions, dim d)
    {
        const uint32_t g = t / kHead, d = t % kHead;
        float o = 0.0f;
        const uint32_t p0 = g * (kWindow / 8), p1 = min(p0 + kWindow / 8, n);
        for (uint32_t p = p0; p < p1; ++p) {
            o = fmaf(e[p], vs[p * kRowStride + d], o);
        }
        part[g][d] = o;
    }
    __syncthreads();
    if (t < uint32_t(kHead) && pos < capacity) {
        const float o = (((part[0][t] + part[1][t]) + (part[2][t] + part[3][t])) +
                         ((part[4][t] + part[5][t]) + (part[6][t] + part[7][t])));
        out[head * kHead + t] = o / den;
    }
}

// Prefill: attention of a run of tokens on f32 MFMA, v_mfma_f32_16x16x4_f32 (D 16x16
// += A 16x4 B 4x16; lane l holds A[l%16][l/16] and B[l/16][l%16] and receives D rows
// 4(l/16)..+3 of column l%16).  One workgroup per (kv head, 16 consecutive tokens):
// the 8 query heads of the group times 16 tokens are 128 queries, in tiles of 16, two
// tiles per wave.  The union of the block's spans streams through LDS in chunks of 64
// positions, each K/V row loaded once per workgroup.  Per chunk and query tile:
//  - S^T (positions x queries) = K Q^T: A is 16 K rows from LDS, B the tile's queries,
//    held in registers for the whole launch; K step (s, j) covers dims 16s + 4k + j for
//    lane group k, so each lane reads its K operands as float4;
//  - an online softmax per query (a column of S^T: the lane's 4 rows of each position
//    tile and the 4 lanes of its column).  m starts at the sink and l at
//    exp(sink - sink) = 1, so the sink takes part in the max and the denominator
//    (model.cpp:270-281); per chunk m' = max(m, scores), and l and O are rescaled by
//    exp(m - m');
//  - O^T (dims x queries) += V^T P^T: K step j of position tile p takes positions
//    16p + 4k + j for lane group k, which is row j of the lane's own S^T tile, so the
//    probabilities never leave their registers; A reads V rows from LDS.
// The output is O / l.
constexpr int kPfTokens = 16;
constexpr int kPfQueries = kPfTokens * kGroup;                // 128
constexpr int kPfThreads = 256;
constexpr int kPfTiles = kPfQueries / 16 / (kPfThreads / 64);  // query tiles per wave: 2

__device__ inline mf::f32x4 mfma_f32(float a, float b, const mf::f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__global__ __launch_bounds__(kPfThreads) void attn_prefill_kernel(const float *__restrict__ q,
                                                                  const float *__restrict__ k_cache,
                                                                  const float *__restrict__ v_cache,
                                                                  const float *__restrict__ sinks, uint32_t first,
                                                                  uint32_t tokens, uint32_t layer_index,
                                                                  float *__restrict__ out) {
    using mf::f32x4;
    __shared__ __attribute__((aligned(16))) float ks[kChunk * kRowStride];
    __shared__ __attribute__((aligned(16))) float vs[kChunk * kRowStride];
    const uint32_t t = threadIdx.x, wave = t / 64, lane = t % 64, n = lane % 16, g = lane / 16;
    const uint32_t kvh = blockIdx.y, block0 = blockIdx.x * kPfTokens;
    const uint32_t last_local = min(block0 + kPfTokens, tokens) - 1;
    // the block's positions: from the first token's span start to the last token
    const uint32_t lo = span_of(first + block0, layer_index).first;
    const uint32_t hi = first + last_local;

    // this lane's query (column n) of each of the wave's tiles
    float qv[kPfTiles][16];  // [4s + j] = Q[dim 16s + 4g + j]
    uint32_t qpos[kPfTiles], qfirst[kPfTiles], qlocal[kPfTiles], qhead[kPfTiles];
    float m[kPfTiles], l[kPfTiles];
    f32x4 o[kPfTiles][4];  // O^T tiles: dims 16M + 4g + i of the query
#pragma unroll
    for (int qi = 0; qi < kPfTiles; ++qi) {
        const uint32_t query = (wave * kPfTiles + qi) * 16 + n;
        qlocal[qi] = block0 + query / kGroup;
        qhead[qi] = kvh * kGroup + query % kGroup;
        const uint32_t lc = min(qlocal[qi], last_local);  // past the last token: a stand-in, not written
        qpos[qi] = first + lc;
        qfirst[qi] = span_of(qpos[qi], layer_index).first;
        const float4 *q4 = reinterpret_cast<const float4 *>(q + (size_t(lc) * kQHeads + qhead[qi]) * kHead);
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
            const float4 v = q4[4 * s4 + g];
            qv[qi][4 * s4] = v.x;
            qv[qi][4 * s4 + 1] = v.y;
            qv[qi][4 * s4 + 2] = v.z;
            qv[qi][4 * s4 + 3] = v.w;
        }
        m[qi] = sinks[qhead[qi]];
        l[qi] = g == 0 ? 1.0f : 0.0f;  // the sink's exp(sink - m), counted once per column
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            o[qi][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }

    constexpr int kPer = kChunk * (kHead / 4) / kPfThreads;  // 4 float4 of K and of V per thread
    for (uint32_t c0 = lo - lo % kChunk; c0 <= hi; c0 += kChunk) {
        __syncthreads();  // the previous chunk's reads are done
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const uint32_t f = t + uint32_t(k) * kPfThreads, p = f / (kHead / 4), d4 = f % (kHead / 4);
            const uint32_t at = min(c0 + p, hi);  // positions past the block's last re-read it
            const size_t row = (size_t(at) * kKvHeads + kvh) * kHead;
            *reinterpret_cast<float4 *>(ks + p * kRowStride + 4 * d4) = reinterpret_cast<const float4 *>(k_cache + row)[d4];
            *reinterpret_cast<float4 *>(vs + p * kRowStride + 4 * d4) = reinterpret_cast<const float4 *>(v_cache + row)[d4];
        }
        __syncthreads();

        // S^T: [query tile][position tile], lane rows 4g..4g+3 = positions 16p + 4g + i
        f32x4 sc[kPfTiles][4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
#pragma unroll
            for (int qi = 0; qi < kPfTiles; ++qi) {
                sc[qi][p] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const float4 a = *reinterpret_cast<const float4 *>(ks + (16 * p + n) * kRowStride + 16 * s4 + 4 * g);
#pragma unroll
                for (int qi = 0; qi < kPfTiles; ++qi) {
                    sc[qi][p] = mfma_f32(a.x, qv[qi][4 * s4], sc[qi][p]);
                }
#pragma unroll
                for (int qi = 0; qi < kPfTiles; ++qi) {
                    sc[qi][p] = mfma_f32(a.y, qv[qi][4 * s4 + 1], sc[qi][p]);
                }
#pragma unroll
                for (int qi = 0; qi < kPfTiles; ++qi) {
                    sc[qi][p] = mfma_f32(a.z, qv[qi][4 * s4 + 2], sc[qi][p]);
                }
#pragma unroll
                for (int qi = 0; qi < kPfTiles; ++qi) {
                    sc[qi][p] = mfma_f32(a.w, qv[qi][4 * s4 + 3], sc[qi][p]);
                }
            }
        }
        // scores (1/sqrt(64) = 0.125, exact), mask, online softmax; sc becomes P^T
#pragma unroll
        for (int qi = 0; qi < kPfTiles; ++qi) {
            float cmax = -INFINITY;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t at = c0 + 16 * p + 4 * g + i;
                    const bool in = at >= qfirst[qi] && at <= qpos[qi];
                    const float s = in ? sc[qi][p][i] * 0.125f : -INFINITY;
                    sc[qi][p][i] = s;
                    cmax = fmaxf(cmax, s);
                }
            }
            cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
            cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
            const float m2 = fmaxf(m[qi], cmax);
            const float scale = expf(m[qi] - m2);
            float lsum = 0.0f;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float s = sc[qi][p][i];
                    const float x = s == -INFINITY ? 0.0f : expf(s - m2);
                    sc[qi][p][i] = x;
                    lsum += x;
                }
            }
            l[qi] = l[qi] * scale + lsum;
            m[qi] = m2;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                o[qi][mt] *= scale;
            }
        }
        // O^T += V^T P^T
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float a = vs[(16 * p + 4 * g + j) * kRowStride + 16 * mt + n];
#pragma unroll
                    for (int qi = 0; qi < kPfTiles; ++qi) {
                        o[qi][mt] = mfma_f32(a, sc[qi][p][j], o[qi][mt]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int qi = 0; qi < kPfTiles; ++qi) {
        float den = l[qi] + __shfl_xor(l[qi], 16);
        den = den + __shfl_xor(den, 32);
        if (qlocal[qi] < tokens) {
            float *dst = out + (size_t(qlocal[qi]) * kQHeads + qhead[qi]) * kHead;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const f32x4 v = o[qi][mt];
                *reinterpret_cast<float4 *>(dst + 16 * mt + 4 * g) =
                    make_float4(v[0] / den, v[1] / den, v[2] / den, v[3] / den);
            }
        }
    }
}

}  // namespace

namespace ttl {
// Workspace floats needed by ttl_attention_decode for a given capacity.
size_t attention_partials_floats(uint32_t capacity) {
    const size_t chunks = (capacity + kChunk - 1) / kChunk;
    return size_t(kQHeads) * chunks * (kHead + 2);
}
}  // namespace ttl

namespace {

// Attention of the token at *position; max_chunks = the chunks the partials of
// one token hold (at least those of its span).
void launch_attention(ttl_ctx *ctx, const float *q, const float *k_cache, const float *v_cache, const float *sinks,
                      const int32_t *position, uint32_t capacity, uint32_t layer_index, uint32_t max_chunks,
                      float *workspace, float *out) {
    if (layer_index % 2 == 0) {
        // the sliding window fits one workgroup per query head
        attn_window_kernel<<<kQHeads, kWinThreads, 0, ctx->stream>>>(q, k_cache, v_cache, sinks, position, capacity,
                                                                     layer_index, out);
        return;
    }
    float *o_part = workspace;
    float2 *ml_part = reinterpret_cast<float2 *>(workspace + size_t(kQHeads) * max_chunks * kHead);
    attn_partial_kernel<<<dim3(max_chunks, kKvHeads), kThreads, 0, ctx->stream>>>(
        q, k_cache, v_cache, position, capacity, layer_index, max_chunks, o_part, ml_part);
    attn_combine_kernel<<<kQHeads, kHead, 0, ctx->stream>>>(o_part, ml_part, sinks, position, capacity, layer_index,
                                                            max_chunks, out);
}


// ---- ttl_attention_decode_noalloc: the partials in a static device array ------------
//
// For callers that cannot allocate (graph capture, serving loops): one array per GPU,
// sized for the largest capacity the kernels take (kMaxCombineChunks chunks of 64
// positions, 16384 positions: 64 x 256 x 66 floats = 4,325,376 bytes), which each GPU
// the library runs on holds until the process ends.  Host code never passes the
// array's name to a kernel: its device address is looked up once per device, with that
// device current, when a context opens (ttl::attention_scratch_init, from ttl_create).
constexpr size_t kScratchFloats = size_t(kQHeads) * kMaxCombineChunks * (kHead + 2);
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
float *g_scratch_ptr[kMaxScratchDevices] = {};

float *scratch_for(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    return device >= 0 && device < kMaxScratchDevices ? g_scratch_ptr[device] : nullptr;
}

}  // namespace

namespace ttl {
int attention_scratch_init(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    TTL_REQUIRE(device >= 0 && device < kMaxScratchDevices, TTL_ERR_NO_DEVICE,
                "ttl_create: device ordinal %d above %d", device, kMaxScratchDevices - 1);
    if (g_scratch_ptr[device]) {
        return TTL_OK;
    }
    void *ptr = nullptr;
    TTL_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    g_scratch_ptr[device] = static_cast<float *>(ptr);
    return TTL_OK;
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
    TTL_REQUIRE(capacity > 0 && capacity <= uint32_t(kMaxCombineChunks * kChunk), TTL_ERR_SHAPE,
                "ttl_attention_decode: capacity must be 1..%d", kMaxCombineChunks * kChunk);
    TTL_REQUIRE(((uintptr_t)q_dev & 15) == 0 && ((uintptr_t)k_cache_dev & 15) == 0 && ((uintptr_t)v_cache_dev & 15) == 0,
                TTL_ERR_INVALID, "ttl_attention_decode: q, k and v must be 16-byte aligned");
    launch_attention(ctx, q_dev, k_cache_dev, v_cache_dev, sinks_dev, position_dev, capacity, layer_index,
                     (capacity + kChunk - 1) / kChunk, workspace_dev, out_dev);
    TTL_LAUNCHED("attention kernels");
    return TTL_OK;
}


int ttl_attention_decode_noalloc(ttl_ctx *ctx, const float *q_dev, const float *k_cache_dev,
                                 const float *v_cache_dev, const float *sinks_dev, const int32_t *position_dev,
                                 uint32_t capacity, uint32_t layer_index, float *out_dev) {
    TTL_REQUIRE(ctx && q_dev && k_cache_dev && v_cache_dev && sinks_dev && position_dev && out_dev, TTL_ERR_INVALID,
                "ttl_attention_decode_noalloc: null argument");
    TTL_REQUIRE(capacity > 0 && capacity <= uint32_t(kMaxCombineChunks * kChunk), TTL_ERR_SHAPE,
                "ttl_attention_decode_noalloc: capacity must be 1..%d (the static partials hold %zu bytes)",
                kMaxCombineChunks * kChunk, kScratchFloats * sizeof(float));
    TTL_REQUIRE(((uintptr_t)q_dev & 15) == 0 && ((uintptr_t)k_cache_dev & 15) == 0 && ((uintptr_t)v_cache_dev & 15) == 0,
                TTL_ERR_INVALID, "ttl_attention_decode_noalloc: q, k and v must be 16-byte aligned");
    float *partials = scratch_for(ctx->device);
    TTL_REQUIRE(partials, TTL_ERR_INVALID, "ttl_attention_decode_noalloc: no static partials on device %d",
                ctx->device);
    const uint32_t chunks = (capacity + kChunk - 1) / kChunk;
    TTL_REQUIRE(ttl::attention_partials_floats(capacity) <= kScratchFloats, TTL_ERR_SHAPE,
                "ttl_attention_decode_noalloc: %u chunks exceed the static partials", chunks);
    launch_attention(ctx, q_dev, k_cache_dev, v_cache_dev, sinks_dev, position_dev, capacity, layer_index, chunks,
                     partials, out_dev);
    TTL_LAUNCHED("attention kernels");
    return TTL_OK;
}

int ttl_attention_prefill(ttl_ctx *ctx, const float *q_dev, const float *k_cache_dev, const float *v_cache_dev,
                          const float *sinks_dev, uint32_t first_position, uint32_t tokens, uint32_t capacity,
                          uint32_t layer_index, float *out_dev) {
    TTL_REQUIRE(ctx && q_dev && k_cache_dev && v_cache_dev && sinks_dev && out_dev, TTL_ERR_INVALID,
                "ttl_attention_prefill: null argument");
    TTL_REQUIRE(capacity > 0 && capacity <= uint32_t(kMaxCombineChunks * kChunk), TTL_ERR_SHAPE,
                "ttl_attention_prefill: capacity must be 1..%d", kMaxCombineChunks * kChunk);
    TTL_REQUIRE(tokens > 0 && tokens <= 65535 && size_t(first_position) + tokens <= capacity, TTL_ERR_SHAPE,
                "ttl_attention_prefill: positions %u..%u do not fit the capacity %u", first_position,
                first_position + tokens - 1, capacity);
    TTL_REQUIRE(((uintptr_t)q_dev & 15) == 0 && ((uintptr_t)k_cache_dev & 15) == 0 && ((uintptr_t)v_cache_dev & 15) == 0,
                TTL_ERR_INVALID, "ttl_attention_prefill: q, k and v must be 16-byte aligned");
    attn_prefill_kernel<<<dim3((tokens + kPfTokens - 1) / kPfTokens, kKvHeads), kPfThreads, 0, ctx->stream>>>(
        q_dev, k_cache_dev, v_cache_dev, sinks_dev, first_position, tokens, layer_index, out_dev);
    TTL_LAUNCHED("attn_prefill_kernel");
    return TTL_OK;
}

}  // extern "C"
