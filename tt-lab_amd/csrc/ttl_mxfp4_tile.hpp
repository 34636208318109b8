// Device building blocks of the MXFP4 matvec kernels (one wave = one 16-row tile).
//
//  - Lane l works on row l%16 of the tile and on blocks kb = 4*i + l/16,
//    i = 0..22, so each 64-lane 16-byte load reads 1 KiB of contiguous codes.
//  - All 23 code chunks and the lane's 24 scale bytes are requested before any
//    arithmetic, so a wave keeps ~23 KiB in flight from HBM.
//  - The activation vector sits in LDS with a padded stride (36 floats per
//    32-value block), so the four distinct addresses of a ds_read_b128 fall in
//    different banks.
//  - Decode happens in registers: v_cvt_scalef32_pk_f32_fp4 turns one byte into
//    the two E2M1 values it holds (low nibble -> element j, high -> j+16); the 32
//    products of a block accumulate in f32 and the block's E8M0 scale is applied
//    once to that partial as an exact power of two (v_ldexp_f32).
//  - The four lanes of a row are combined with two cross-lane exchanges.
#pragma once

#include "ttl_internal.hpp"

namespace mxt {

constexpr int x_stride = 36;                       // padded LDS floats per block
constexpr int x_blocks = mx::iters * mx::lanes_k;  // 92: blocks 90 and 91 are zero
constexpr int x_floats = x_blocks * x_stride;

template <int Sel>
__device__ inline float2 cvt_fp4x2(uint32_t word) {
    // The two E2M1 values of byte Sel of `word`: .x from the low nibble, .y from the high.
    const auto v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, Sel);
    return make_float2(v[0], v[1]);
}

// Unscaled dot product of one block's 32 codes with x[0..31] of the block.
__device__ inline float block_dot(const uint4 c, const float *__restrict__ xb) {
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
    float lo = 0.0f, hi = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 xl = *reinterpret_cast<const float4 *>(xb + 4 * q);
        const float4 xh = *reinterpret_cast<const float4 *>(xb + 16 + 4 * q);
        const float2 v0 = cvt_fp4x2<0>(w[q]);
        const float2 v1 = cvt_fp4x2<1>(w[q]);
        const float2 v2 = cvt_fp4x2<2>(w[q]);
        const float2 v3 = cvt_fp4x2<3>(w[q]);
        lo = fmaf(v0.x, xl.x, lo);
        hi = fmaf(v0.y, xh.x, hi);
        lo = fmaf(v1.x, xl.y, lo);
        hi = fmaf(v1.y, xh.y, hi);
        lo = fmaf(v2.x, xl.z, lo);
        hi = fmaf(v2.y, xh.z, hi);
        lo = fmaf(v3.x, xl.w, lo);
        hi = fmaf(v3.y, xh.w, hi);
    }
    return lo + hi;
}

// Copies x (2880 floats, 16-byte aligned) into the padded LDS layout; the two
// padding blocks are zero.  All threads of the workgroup take part.
__device__ inline void stage_x(const float *__restrict__ x, float *xs) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    for (int i = threadIdx.x; i < x_blocks * 8; i += blockDim.x) {
        const int block = i / 8, part = i % 8;
        const float4 v = block < mx::blocks ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        *reinterpret_cast<float4 *>(xs + block * x_stride + part * 4) = v;
    }
}

// Registers of one lane for one tile: its 23 code chunks and 24 scale bytes.
struct TileRegs {
    uint4 q[mx::iters];
    uint32_t sw[6];
};

// Issues all of the lane's loads for one tile.  Callers issue their x loads
// first, so that finishing the staging waits for those alone.
__device__ __attribute__((always_inline)) inline void tile_load(const uint8_t *__restrict__ codes,
                                                                const uint8_t *__restrict__ scales,
                                                                size_t tile_index, uint32_t lane, TileRegs &regs) {
    const uint32_t r = lane % mx::tile_rows;
    const uint32_t kl = lane / mx::tile_rows;
    const uint4 *tc = reinterpret_cast<const uint4 *>(codes) + tile_index * mx::blocks * mx::tile_rows + r;
    const uint2 *ts = reinterpret_cast<const uint2 *>(scales + tile_index * mx::tile_scale_bytes +
                                                      size_t(lane) * mx::scale_pad);
    const uint2 s01 = ts[0], s23 = ts[1], s45 = ts[2];
    regs.sw[0] = s01.x;
    regs.sw[1] = s01.y;
    regs.sw[2] = s23.x;
    regs.sw[3] = s23.y;
    regs.sw[4] = s45.x;
    regs.sw[5] = s45.y;
    // Unconditional loads (no branch, so the compiler can wait for them one by one
    // as the compute consumes them): the last iteration's lanes for blocks 90 and 91
    // read the next tile or the tensor's zero tail; their x is zero.
    // Issued in iteration order (the scheduler may not reorder them), so that the
    // compute can wait for each chunk alone as it arrives.  Blocks 90 and 91 of the
    // last iteration re-read block 89 (zero x there).
#pragma unroll
    for (int i = 0; i < mx::iters; ++i) {
        regs.q[i] = ttl::load_stream(tc + size_t(min(uint32_t(4 * i) + kl, uint32_t(mx::blocks - 1))) * mx::tile_rows);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Dot products of the tile's 16 rows with x (in LDS).  The row sum for row
// lane%16 is returned in every lane (lanes l, l+16, l+32, l+48 agree).
__device__ __attribute__((always_inline)) inline float tile_compute(const TileRegs &regs, const float *xs,
                                                                   uint32_t lane) {
    const uint32_t kl = lane / mx::tile_rows;
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < mx::iters; ++i) {
        const uint32_t kb = 4 * i + kl;
        const int e8 = int((regs.sw[i / 4] >> (8 * (i % 4))) & 0xffu);
        acc += __builtin_amdgcn_ldexpf(block_dot(regs.q[i], xs + kb * x_stride), e8 - 127);
    }
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    return acc;
}

// ---- split-K: W waves share one tile ----------------------------------------
//
// Wave w of a tile takes iterations [w*P, w*P + P), P = ceil(23 / W), so the
// per-wave dependency chain (and the time the last wave of a SIMD computes after
// its data arrived) shrinks W-fold.  Iterations past 22 read blocks 92.. of the
// padded layout: zero x in LDS, scale byte 127, codes from the next tile or the
// tensor's zero tail, so they add exactly zero.
template <int W>
struct Split {
    static constexpr int per = (mx::iters + W - 1) / W;   // iterations per wave
    static constexpr int x_blocks = per * W * mx::lanes_k;  // staged x blocks (zero padded)
    static constexpr int x_floats = x_blocks * x_stride;
    static_assert(per % 2 == 0 && per * W <= mx::scale_pad, "scale bytes are read in pairs from the lane record");
};

template <int W>
struct SplitRegs {
    uint4 q[Split<W>::per];
    uint32_t s[Split<W>::per / 2];  // the wave's scale bytes, two per word (low halves)
};

// Issues wave w's loads for one tile: its scale bytes first (every iteration
// needs them), then its code chunks in iteration order.
template <int W>
__device__ __attribute__((always_inline)) inline void split_load(const uint8_t *__restrict__ codes,
                                                                 const uint8_t *__restrict__ scales,
                                                                 size_t tile_index, uint32_t w, uint32_t lane,
                                                                 SplitRegs<W> &regs) {
    constexpr int P = Split<W>::per;
    const uint32_t r = lane % mx::tile_rows;
    const uint32_t kl = lane / mx::tile_rows;
    const uint16_t *ts = reinterpret_cast<const uint16_t *>(scales + tile_index * mx::tile_scale_bytes +
                                                            size_t(lane) * mx::scale_pad + w * P);
#pragma unroll
    for (int j = 0; j < P / 2; ++j) {
        regs.s[j] = ts[j];
    }
    const uint4 *tc = reinterpret_cast<const uint4 *>(codes) + tile_index * mx::blocks * mx::tile_rows + r;
#pragma unroll
    for (int j = 0; j < P; ++j) {
        // blocks past the row end re-read block 89 (same address as another lane of
        // the load: no extra memory traffic); their x is zero
        const uint32_t kb = min(uint32_t(4 * (w * P + j)) + kl, uint32_t(mx::blocks - 1));
        regs.q[j] = ttl::load_stream(tc + size_t(kb) * mx::tile_rows);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Wave w's partial dot products for the tile's 16 rows (row lane%16 in every lane).
template <int W>
__device__ __attribute__((always_inline)) inline float split_compute(const SplitRegs<W> &regs, const float *xs,
                                                                    uint32_t w, uint32_t lane) {
    constexpr int P = Split<W>::per;
    const uint32_t kl = lane / mx::tile_rows;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < P; ++j) {
        const uint32_t kb = 4 * (w * P + j) + kl;
        const int e8 = int((regs.s[j / 2] >> (8 * (j % 2))) & 0xffu);
        acc += __builtin_amdgcn_ldexpf(block_dot(regs.q[j], xs + kb * x_stride), e8 - 127);
    }
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    return acc;
}

}  // namespace mxt
