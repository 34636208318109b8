// Device generators for synthetic inputs.  They implement the specification
// written in oracle/ttlab_oracle.h bit for bit (integer hashing; the one float
// rounding is an int->float conversion and an explicit, unfused multiply-add).
#include "ttl_internal.hpp"

namespace {

__device__ inline float unit_normal(uint64_t seed, uint64_t stream, uint64_t i) {
    int32_t sum = 0;
#pragma unroll
    for (uint64_t j = 0; j < 12; ++j) {
        sum += int32_t(synth::hash(seed, stream, 12 * i + j) >> 40);
    }
    sum -= 6 << 24;
    return float(sum) * 0x1p-24f;
}

__device__ inline uint16_t f32_to_bf16_rne(float value) {
    uint32_t bits = __float_as_uint(value);
    const uint32_t lsb = (bits >> 16) & 1u;
    bits += 0x7fffu + lsb;
    return uint16_t(bits >> 16);
}

__global__ void normal_kernel(uint64_t seed, uint64_t stream, size_t offset, size_t n, float mean, float sigma,
                              int bf16, float *out) {
#pragma clang fp contract(off)
    const size_t k = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (k >= n) {
        return;
    }
    const float z = unit_normal(seed, stream, offset + k) * sigma;
    if (bf16) {
        out[k] = __uint_as_float(uint32_t(f32_to_bf16_rne(z)) << 16);
    } else {
        out[k] = mean + z;
    }
}

__device__ inline void mxfp4_block(uint64_t seed, uint64_t stream, uint64_t b, uint32_t emin, uint32_t span,
                                   uint8_t *scale, uint4 *codes) {
    *scale = uint8_t(emin + synth::hash(seed, stream, 3 * b) % span);
    const uint64_t lo = synth::hash(seed, stream, 3 * b + 1);
    const uint64_t hi = synth::hash(seed, stream, 3 * b + 2);
    *codes = make_uint4(uint32_t(lo), uint32_t(lo >> 32), uint32_t(hi), uint32_t(hi >> 32));
}

__global__ void mxfp4_gguf_kernel(uint64_t seed, uint64_t stream, size_t block_offset, size_t n, uint32_t emin,
                                  uint32_t span, uint8_t *out) {
    const size_t k = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (k >= n) {
        return;
    }
    uint8_t scale;
    uint4 codes;
    mxfp4_block(seed, stream, block_offset + k, emin, span, &scale, &codes);
    uint8_t *dst = out + k * 17;
    dst[0] = scale;
    const uint32_t words[4] = {codes.x, codes.y, codes.z, codes.w};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        dst[1 + i] = uint8_t(words[i / 4] >> (8 * (i % 4)));
    }
}

// BF16 bits: random sign and mantissa, exponent uniform in 120..123 (orc_synth_bf16).
__global__ void bf16_kernel(uint64_t seed, uint64_t stream, size_t offset, size_t n, uint16_t *out) {
    const size_t k = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (k >= n) {
        return;
    }
    const uint64_t i = offset + k;
    const uint32_t h = uint32_t(synth::hash(seed, stream, i >> 2) >> (16 * (i & 3))) & 0xffffu;
    out[k] = uint16_t((h & 0x807fu) | ((120u + ((h >> 7) & 3u)) << 7));
}

// Writes expert e (stream + e) straight into the repacked planes.
__global__ void mxfp4_repacked_kernel(uint64_t seed, uint64_t stream, uint32_t rows, uint32_t experts,
                                      uint32_t emin, uint32_t span, uint4 *codes, uint8_t *scales) {
    const size_t gid = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t per_expert = size_t(rows) * mx::blocks;
    if (gid >= per_expert * experts) {
        return;
    }
    const uint32_t e = uint32_t(gid / per_expert);
    const size_t b = gid % per_expert;  // GGUF block index within the expert
    const uint32_t row = uint32_t(b / mx::blocks);
    const uint32_t block = uint32_t(b % mx::blocks);
    uint8_t scale;
    uint4 code;
    mxfp4_block(seed, stream + e, b, emin, span, &scale, &code);
    const size_t tile_index = size_t(e) * (rows / mx::tile_rows) + row / mx::tile_rows;
    codes[mx::code_chunk(tile_index, block, row % mx::tile_rows)] = code;
    scales[mx::scale_offset(tile_index, block, row % mx::tile_rows)] = scale;
}

}  // namespace

namespace ttl {
int synth_mxfp4_repacked(ttl_ctx *ctx, ttl_mxfp4 *t, uint64_t seed, uint64_t stream, uint32_t emin, uint32_t emax) {
    const size_t n = size_t(t->rows) * mx::blocks * t->experts;
    mxfp4_repacked_kernel<<<blocks_for(n, 256), 256, 0, ctx->stream>>>(seed, stream, t->rows, t->experts, emin,
                                                                        emax - emin + 1, (uint4 *)t->codes,
                                                                        t->scales);
    TTL_LAUNCHED("mxfp4_repacked_kernel");
    return TTL_OK;
}
}  // namespace ttl

extern "C" {

int ttl_synth_normal(ttl_ctx *ctx, uint64_t seed, uint64_t stream, size_t offset, size_t n, float mean, float sigma,
                     float *out_dev) {
    TTL_REQUIRE(ctx && (n == 0 || out_dev), TTL_ERR_INVALID, "ttl_synth_normal: null argument");
    if (n) {
        normal_kernel<<<ttl::blocks_for(n, 256), 256, 0, ctx->stream>>>(seed, stream, offset, n, mean, sigma, 0,
                                                                         out_dev);
        TTL_LAUNCHED("normal_kernel");
    }
    return TTL_OK;
}

int ttl_synth_normal_bf16(ttl_ctx *ctx, uint64_t seed, uint64_t stream, size_t offset, size_t n, float sigma,
                          float *out_dev) {
    TTL_REQUIRE(ctx && (n == 0 || out_dev), TTL_ERR_INVALID, "ttl_synth_normal_bf16: null argument");
    if (n) {
        normal_kernel<<<ttl::blocks_for(n, 256), 256, 0, ctx->stream>>>(seed, stream, offset, n, 0.0f, sigma, 1,
                                                                         out_dev);
        TTL_LAUNCHED("normal_kernel");
    }
    return TTL_OK;
}

int ttl_synth_bf16(ttl_ctx *ctx, uint64_t seed, uint64_t stream, size_t offset, size_t n, uint16_t *out_dev) {
    TTL_REQUIRE(ctx && (n == 0 || out_dev), TTL_ERR_INVALID, "ttl_synth_bf16: null argument");
    if (n) {
        bf16_kernel<<<ttl::blocks_for(n, 256), 256, 0, ctx->stream>>>(seed, stream, offset, n, out_dev);
        TTL_LAUNCHED("bf16_kernel");
    }
    return TTL_OK;
}

int ttl_synth_mxfp4_gguf(ttl_ctx *ctx, uint64_t seed, uint64_t stream, size_t block_offset, size_t n,
                         uint32_t emin, uint32_t emax, uint8_t *out_dev) {
    TTL_REQUIRE(ctx && (n == 0 || out_dev), TTL_ERR_INVALID, "ttl_synth_mxfp4_gguf: null argument");
    TTL_REQUIRE(emin <= emax && emax <= 255, TTL_ERR_INVALID, "ttl_synth_mxfp4_gguf: bad exponent range");
    if (n) {
        mxfp4_gguf_kernel<<<ttl::blocks_for(n, 256), 256, 0, ctx->stream>>>(seed, stream, block_offset, n, emin,
                                                                             emax - emin + 1, out_dev);
        TTL_LAUNCHED("mxfp4_gguf_kernel");
    }
    return TTL_OK;
}

}  // extern "C"
