// Device building blocks of the Q8_0 matvec kernels.
//
// Layout (repacked on upload from GGUF Q8_0 rows of 34-byte blocks, fp16 scale
// then 32 int8, tensor.cpp:94-114): a tile is 16 rows; a block's 32 codes are two
// 16-byte halves, ordered [tile][block][half][row], so each of a lane's two loads
// covers whole 256-byte runs across the wave (16 rows x 16 bytes per block, four
// blocks) and can be marked non-temporal; scales are fp16 ordered so each lane's
// scales are contiguous, [tile][block%4][row][block/4 padded].
//
// Work split: one workgroup of 4 waves owns one tile.  Lane l handles row l%16
// and blocks 4*i + l/16; wave w handles iterations i in [w*P, w*P + P), so the
// per-wave dependency chain is a quarter of the row and the tile's four partial
// sums are added in LDS in wave order (deterministic).
//
// Decode: the 32 int8 codes are biased to unsigned (xor 0x80), converted with
// v_cvt_f32_ubyte{0..3} and accumulated against x; the bias is removed with the
// block sum of x: sum_j q_j x_j = sum_j (q_j + 128) x_j - 128 * sum_j x_j.
#pragma once

#include "ttl_internal.hpp"
#include "ttl_stage.hpp"

namespace q8 {

constexpr int tile_rows = 16;
constexpr int lanes_k = 4;
constexpr int waves = 4;

template <int K>
struct Shape {
    static constexpr int blocks = K / 32;
    static constexpr int iters = (blocks + lanes_k - 1) / lanes_k;
    static constexpr int per_wave = (iters + waves - 1) / waves;
    static constexpr int scale_pad = per_wave * waves;  // fp16 scales per lane
    // x blocks staged: every block any wave's iterations touch; blocks past the row
    // end are zero, so padding iterations add exactly zero (their scale is zero too)
    static constexpr int x_blocks = scale_pad * lanes_k;
    static constexpr size_t tile_code_bytes = size_t(blocks) * tile_rows * 32;
    static constexpr size_t tile_scales = size_t(lanes_k) * tile_rows * scale_pad;
};

__host__ __device__ inline int blocks_of(int cols) {
    return cols / 32;
}
__host__ __device__ inline int scale_pad_of(int cols) {
    const int iters = (cols / 32 + lanes_k - 1) / lanes_k;
    return ((iters + waves - 1) / waves) * waves;
}
// Zero bytes after the last tile: lanes of iterations past the last block read there
// unconditionally (their scale is zero).
__host__ __device__ inline size_t tail_pad_bytes(int cols) {
    const int iters = (cols / 32 + lanes_k - 1) / lanes_k;
    const int covered = ((iters + waves - 1) / waves) * waves * lanes_k;
    return size_t(covered - cols / 32) * tile_rows * 32;
}
// fp16 scales per row of the row-major copy used by the batched matmul: the blocks
// rounded up to a multiple of 4 (zero padding), so a quad's four are one 8-byte load.
__host__ __device__ inline int row_scale_stride(int cols) {
    return (cols / 32 + 3) / 4 * 4;
}
// Byte offset of codes 16 h .. 16 h + 15 of (tile, block, row).
__host__ __device__ inline size_t code_offset(size_t tile, uint32_t block, uint32_t half, uint32_t row, int cols) {
    return ((tile * blocks_of(cols) + block) * 2 + half) * (tile_rows * 16) + row * 16;
}
__host__ __device__ inline size_t scale_index(size_t tile, uint32_t block, uint32_t row, int cols) {
    const int pad = scale_pad_of(cols);
    return tile * lanes_k * tile_rows * pad + (size_t(block % lanes_k) * tile_rows + row) * pad + block / lanes_k;
}

// A tile's K range split over W waves (W divides the padded iteration count, which
// the layout fixes at scale_pad): wave w takes iterations [w*PW, w*PW + PW).
template <int K, int W>
struct Split {
    static constexpr int per_wave = Shape<K>::scale_pad / W;
    static_assert(Shape<K>::scale_pad % W == 0, "the split must divide the padded iterations");
    static_assert(per_wave % 2 == 0, "scales are loaded in fp16 pairs");
};

template <int K, int W = waves>
struct TileRegs {
    uint4 c[Split<K, W>::per_wave][2];
    uint32_t s[Split<K, W>::per_wave / 2];  // fp16 scales, two per word
};

// Issues the loads of wave `wave`'s share of one tile.
template <int K, int W = waves>
__device__ __attribute__((always_inline)) inline void tile_load(const uint8_t *__restrict__ codes,
                                                                const uint16_t *__restrict__ scales, size_t tile,
                                                                uint32_t wave, uint32_t lane, TileRegs<K, W> &regs) {
    using S = Shape<K>;
    constexpr int PW = Split<K, W>::per_wave;
    const uint32_t r = lane % tile_rows, kl = lane / tile_rows;
    const uint16_t *sp = scales + tile * S::tile_scales + (size_t(kl) * tile_rows + r) * S::scale_pad + wave * PW;
    // the lane's per-wave fp16 scales are contiguous; loaded first, since every
    // iteration needs them
    const uint32_t *s32 = reinterpret_cast<const uint32_t *>(sp);
#pragma unroll
    for (int j = 0; j < PW / 2; ++j) {
        regs.s[j] = s32[j];
    }
    // Unconditional loads (see tail_pad_bytes): blocks past the row end have a zero
    // scale in the padded scale layout, so their codes contribute nothing.
#pragma unroll
    for (int j = 0; j < PW; ++j) {
        // blocks past the row end re-read the last block (a duplicate address within the
        // load, so no extra memory traffic); their scale is zero
        const int i = int(wave) * PW + j;
        const uint32_t kb = min(uint32_t(4 * i) + kl, uint32_t(S::blocks - 1));
        const uint4 *p = reinterpret_cast<const uint4 *>(codes + ((tile * S::blocks + kb) * 2 * tile_rows + r) * 16);
        regs.c[j][0] = ttl::load_stream(p);
        regs.c[j][1] = ttl::load_stream(p + tile_rows);
        __builtin_amdgcn_sched_barrier(0);  // keep the issue order (see the compute)
    }
}

__device__ inline float block_dot(const uint4 c0, const uint4 c1, const float *__restrict__ xb, float xsum) {
    const uint32_t w[8] = {c0.x ^ 0x80808080u, c0.y ^ 0x80808080u, c0.z ^ 0x80808080u, c0.w ^ 0x80808080u,
                           c1.x ^ 0x80808080u, c1.y ^ 0x80808080u, c1.z ^ 0x80808080u, c1.w ^ 0x80808080u};
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const float4 x = *reinterpret_cast<const float4 *>(xb + 4 * q);
        a0 = fmaf(float(w[q] & 0xffu), x.x, a0);
        a1 = fmaf(float((w[q] >> 8) & 0xffu), x.y, a1);
        a0 = fmaf(float((w[q] >> 16) & 0xffu), x.z, a0);
        a1 = fmaf(float(w[q] >> 24), x.w, a1);
    }
    return fmaf(-128.0f, xsum, a0 + a1);
}

// Wave's partial dot products for the tile's 16 rows; valid in lanes 0..15.
template <int K, int W = waves>
__device__ __attribute__((always_inline)) inline float tile_compute(const TileRegs<K, W> &regs, uint32_t wave,
                                                                   uint32_t lane, const float *xs,
                                                                   const float *xsum) {
    constexpr int PW = Split<K, W>::per_wave;
    const uint32_t kl = lane / tile_rows;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < PW; ++j) {
        // no bounds test: padding iterations have zero x and a zero scale
        const int i = int(wave) * PW + j;
        const uint32_t kb = 4 * i + kl;
        const uint16_t bits = uint16_t(regs.s[j / 2] >> (16 * (j % 2)));
        const float d = __half2float(__ushort_as_half(bits));
        acc = fmaf(d, block_dot(regs.c[j][0], regs.c[j][1], xs + kb * stage::x_stride, xsum[kb]), acc);
    }
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    return acc;
}

// Per-block sums of x (in the padded LDS layout), one thread per block.
__device__ inline void block_sums(const float *xs, uint32_t x_blocks, float *xsum) {
    for (uint32_t b = threadIdx.x; b < x_blocks; b += blockDim.x) {
        const float *p = xs + b * stage::x_stride;
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            s += p[j];
        }
        xsum[b] = s;
    }
    __syncthreads();
}

}  // namespace q8
