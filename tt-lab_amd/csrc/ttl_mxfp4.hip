// MXFP4 tensors (GGUF block layout in, repacked planes on the device) and the
// expert-indexed MXFP4 matvec.  The per-tile inner loop is in ttl_mxfp4_tile.hpp.
#include "ttl_mfma.hpp"
#include "ttl_mxfp4_tile.hpp"
#include "ttl_stage.hpp"

#include <cmath>
#include <vector>

namespace ttl {
int synth_mxfp4_repacked(ttl_ctx *ctx, ttl_mxfp4 *t, uint64_t seed, uint64_t stream, uint32_t emin, uint32_t emax);
}

namespace {


// ---- layout conversion ------------------------------------------------------

__global__ void repack_kernel(const uint8_t *__restrict__ gguf, uint32_t rows, uint32_t experts,
                              uint4 *__restrict__ codes, uint8_t *__restrict__ scales,
                              uint32_t *__restrict__ edge_flag) {
    const size_t gid = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t per_expert = size_t(rows) * mx::blocks;
    if (gid >= per_expert * experts) {
        return;
    }
    const uint32_t e = uint32_t(gid / per_expert);
    const size_t b = gid % per_expert;
    const uint32_t row = uint32_t(b / mx::blocks);
    const uint32_t block = uint32_t(b % mx::blocks);
    const uint8_t *src = gguf + gid * 17;
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        w[i / 4] |= uint32_t(src[1 + i]) << (8 * (i % 4));
    }
    const size_t tile_index = size_t(e) * (rows / mx::tile_rows) + row / mx::tile_rows;
    codes[mx::code_chunk(tile_index, block, row % mx::tile_rows)] = make_uint4(w[0], w[1], w[2], w[3]);
    const uint8_t e8 = src[0];
    scales[mx::scale_offset(tile_index, block, row % mx::tile_rows)] = e8;
    // E8M0 255, or 0 with a code of nonzero magnitude (zero codes decode to 0 at any
    // finite scale): the bf16 MFMA decode cannot represent the block (bit 0); a nonzero
    // block outside the f16 decode's exact range (bit 1)
    const bool nonzero = ((w[0] | w[1] | w[2] | w[3]) & 0x77777777u) != 0;
    const uint32_t flags = ((e8 == 255 || (e8 == 0 && nonzero)) ? 1u : 0u) |
                           ((nonzero && (e8 < mf::f16_scale_min || e8 > mf::f16_scale_max)) ? 2u : 0u);
    if (flags) {
        atomicOr(&edge_flag[e], flags);
    }
}

__global__ void unpack_kernel(const uint4 *__restrict__ codes, const uint8_t *__restrict__ scales, uint32_t rows,
                              uint32_t experts, uint8_t *__restrict__ gguf) {
    const size_t gid = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t per_expert = size_t(rows) * mx::blocks;
    if (gid >= per_expert * experts) {
        return;
    }
    const uint32_t e = uint32_t(gid / per_expert);
    const size_t b = gid % per_expert;
    const uint32_t row = uint32_t(b / mx::blocks);
    const uint32_t block = uint32_t(b % mx::blocks);
    const size_t tile_index = size_t(e) * (rows / mx::tile_rows) + row / mx::tile_rows;
    const uint4 c = codes[mx::code_chunk(tile_index, block, row % mx::tile_rows)];
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
    uint8_t *dst = gguf + gid * 17;
    dst[0] = scales[mx::scale_offset(tile_index, block, row % mx::tile_rows)];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        dst[1 + i] = uint8_t(w[i / 4] >> (8 * (i % 4)));
    }
}

// ---- decode ------------------------------------------------------------------

// tensor.cpp:34: the reference's integer for code c (twice its E2M1 value).
__device__ inline int mxfp4_int(uint32_t code) {
    const uint32_t m = code & 7u;
    const int magnitude = m < 4 ? int(m) : int(((m & 1u) ? 3u : 2u) << ((m >> 1) - 1));
    return (code & 8u) ? -magnitude : magnitude;
}

// tensor.cpp:36-44: 2^(e-128) from its bit pattern.
__device__ inline float mxfp4_scale(uint32_t e) {
    const uint32_t bits = e < 2 ? (0x00200000u << e) : ((e - 1u) << 23);
    return __uint_as_float(bits);
}

__global__ void dequant_kernel(const uint4 *__restrict__ codes, const uint8_t *__restrict__ scales, uint32_t rows,
                               uint32_t expert, int mode, float *__restrict__ out) {
    const size_t gid = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= size_t(rows) * mx::blocks) {
        return;
    }
    const uint32_t row = uint32_t(gid / mx::blocks);
    const uint32_t block = uint32_t(gid % mx::blocks);
    const size_t tile_index = size_t(expert) * (rows / mx::tile_rows) + row / mx::tile_rows;
    const uint4 c = codes[mx::code_chunk(tile_index, block, row % mx::tile_rows)];
    const uint32_t e = scales[mx::scale_offset(tile_index, block, row % mx::tile_rows)];
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
    float *dst = out + size_t(row) * mx::cols + block * 32;
    if (mode == 0) {
        const float scale = mxfp4_scale(e);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t byte = (w[j / 4] >> (8 * (j % 4))) & 0xffu;
            dst[j] = scale * float(mxfp4_int(byte & 15u));
            dst[j + 16] = scale * float(mxfp4_int(byte >> 4));
        }
    } else if (mode == 2) {
        // the prefill kernels' decode: bf16 = E2M1 x 2^(e-127) straight from the
        // gfx950 conversion with the E8M0 scale (ttl_mfma.hpp), widened to f32
        const float scale = mf::e8m0_scale(e);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const mf::bf16x8 v = mf::decode_step(w[q], scale);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                dst[4 * q + b] = float(v[2 * b]);
                dst[4 * q + b + 16] = float(v[2 * b + 1]);
            }
        }
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float2 v0 = mxt::cvt_fp4x2<0>(w[q]);
            const float2 v1 = mxt::cvt_fp4x2<1>(w[q]);
            const float2 v2 = mxt::cvt_fp4x2<2>(w[q]);
            const float2 v3 = mxt::cvt_fp4x2<3>(w[q]);
            const int k = int(e) - 127;
            dst[4 * q + 0] = __builtin_amdgcn_ldexpf(v0.x, k);
            dst[4 * q + 16] = __builtin_amdgcn_ldexpf(v0.y, k);
            dst[4 * q + 1] = __builtin_amdgcn_ldexpf(v1.x, k);
            dst[4 * q + 17] = __builtin_amdgcn_ldexpf(v1.y, k);
            dst[4 * q + 2] = __builtin_amdgcn_ldexpf(v2.x, k);
            dst[4 * q + 18] = __builtin_amdgcn_ldexpf(v2.y, k);
            dst[4 * q + 3] = __builtin_amdgcn_ldexpf(v3.x, k);
            dst[4 * q + 19] = __builtin_amdgcn_ldexpf(v3.y, k);
        }
    }
}

// ---- matvec ------------------------------------------------------------------

// One workgroup per (slot, 16-row tile) of the expert selected for the slot
// (expert_ids[slot], or expert_base + slot without ids: no dependent load): twelve
// waves split the tile's K range (two 128-column iterations each, so the decode and
// FMAs left after a wave's last load arrives are a twelfth of the row; 4.63-4.70 -> 4.47 us
// per 5760-row launch against four waves), and their partial sums are added in wave
// order.  The x loads are issued first, then the weight loads, all unconditionally: an
// invalid expert reads expert 0 and its rows become NaN.
constexpr int kMvSplit = 12;
using MvSplit = mxt::Split<kMvSplit>;

__global__ __launch_bounds__(kMvSplit * 64) void matvec_kernel(
    const uint8_t *__restrict__ codes, const uint8_t *__restrict__ scales, uint32_t rows, uint32_t tiles,
    uint32_t experts, const float *__restrict__ bias, const float *__restrict__ x, uint32_t x_stride,
    const int32_t *__restrict__ expert_ids, uint32_t expert_base, float *__restrict__ y) {
    __shared__ __attribute__((aligned(16))) float xs[MvSplit::x_floats];
    __shared__ float red[stage::red_floats(MvSplit::x_blocks)];
    __shared__ float part[kMvSplit][mx::tile_rows];
    const uint32_t slot = blockIdx.x / tiles, tile = blockIdx.x % tiles;
    const uint32_t w = threadIdx.x / 64, lane = threadIdx.x % 64;

    stage::Input in{};
    in.base = x + size_t(slot) * x_stride;
    stage::Pending<mx::cols, MvSplit::x_blocks, kMvSplit * 64, stage::kPlain> pending;
    stage::stage_load(in, pending);
    const int32_t e = expert_ids ? expert_ids[slot] : int32_t(expert_base + slot);
    const bool valid = e >= 0 && uint32_t(e) < experts;
    const uint32_t e_safe = valid ? uint32_t(e) : 0u;
    const uint32_t row = tile * mx::tile_rows + lane % mx::tile_rows;
    const float bv = bias ? bias[size_t(e_safe) * rows + row] : 0.0f;
    mxt::SplitRegs<kMvSplit> regs;
    mxt::split_load<kMvSplit>(codes, scales, size_t(e_safe) * tiles + tile, w, lane, regs);
    stage::stage_finish(in, pending, xs, red);
    const float acc = mxt::split_compute<kMvSplit>(regs, xs, w, lane);
    if (lane < mx::tile_rows) {
        part[w][lane] = acc;
    }
    __syncthreads();
    if (threadIdx.x < uint32_t(mx::tile_rows)) {
        float sum = part[0][threadIdx.x];
#pragma unroll
        for (int k = 1; k < kMvSplit; ++k) {
            sum += part[k][threadIdx.x];
        }
        y[size_t(slot) * rows + row] = valid ? (bias ? sum + bv : sum) : __builtin_nanf("");
    }
}

int check_tensor(const ttl_mxfp4 *t, const char *who) {
    TTL_REQUIRE(t && t->codes && t->scales, TTL_ERR_INVALID, "%s: null tensor", who);
    return TTL_OK;
}

int alloc_tensor(ttl_ctx *ctx, uint32_t rows, uint32_t cols, uint32_t experts, ttl_mxfp4 **out, const char *who) {
    TTL_REQUIRE(ctx && out, TTL_ERR_INVALID, "%s: null argument", who);
    *out = nullptr;
    TTL_REQUIRE(cols == uint32_t(mx::cols), TTL_ERR_SHAPE, "%s: cols must be %d (got %u)", who, mx::cols, cols);
    TTL_REQUIRE(rows > 0 && rows % mx::tile_rows == 0, TTL_ERR_SHAPE, "%s: rows must be a positive multiple of %d",
                who, mx::tile_rows);
    TTL_REQUIRE(experts > 0, TTL_ERR_SHAPE, "%s: experts must be positive", who);
    ttl_mxfp4 *t = new ttl_mxfp4;
    t->rows = rows;
    t->cols = cols;
    t->experts = experts;
    t->tiles = rows / mx::tile_rows;
    const size_t tiles_total = size_t(t->tiles) * experts;
    t->code_bytes = tiles_total * mx::tile_code_bytes;
    t->scale_bytes = tiles_total * mx::tile_scale_bytes;
    hipError_t err = hipMalloc(&t->codes, t->code_bytes + mx::tail_pad_bytes);
    if (err == hipSuccess) {
        err = hipMalloc(&t->scales, t->scale_bytes + mx::edge_flag_bytes(experts));
    }
    if (err != hipSuccess) {
        (void)hipFree(t->codes);
        delete t;
        return ttl::hip_fail(err, who);
    }
    // Padding scale bytes must decode to a finite scale (their blocks are zero).
    int rc = ttl_fill_bytes(ctx, t->scales, mx::pad_scale, t->scale_bytes);
    if (rc == TTL_OK) {
        rc = ttl_fill_bytes(ctx, t->scales + t->scale_bytes, 0, mx::edge_flag_bytes(experts));
    }
    if (rc == TTL_OK) {
        rc = ttl_fill_bytes(ctx, t->codes + t->code_bytes, 0, mx::tail_pad_bytes);
    }
    if (rc != TTL_OK) {
        ttl_mxfp4_free(ctx, t);
        return rc;
    }
    *out = t;
    return TTL_OK;
}

}  // namespace

extern "C" {

int ttl_mxfp4_upload_dev(ttl_ctx *ctx, const void *gguf_blocks_dev, uint32_t rows, uint32_t cols,
                         uint32_t experts, ttl_mxfp4 **out) {
    TTL_REQUIRE(gguf_blocks_dev, TTL_ERR_INVALID, "ttl_mxfp4_upload_dev: null blocks");
    int rc = alloc_tensor(ctx, rows, cols, experts, out, "ttl_mxfp4_upload_dev");
    if (rc != TTL_OK) {
        return rc;
    }
    ttl_mxfp4 *t = *out;
    const size_t n = size_t(rows) * mx::blocks * experts;
    uint32_t *flag = reinterpret_cast<uint32_t *>(t->scales + t->scale_bytes);
    repack_kernel<<<ttl::blocks_for(n, 256), 256, 0, ctx->stream>>>((const uint8_t *)gguf_blocks_dev, rows, experts,
                                                                     (uint4 *)t->codes, t->scales, flag);
    hipError_t err = hipGetLastError();
    std::vector<uint32_t> edge(experts, 0u);
    if (err == hipSuccess) {
        err = hipMemcpyAsync(edge.data(), flag, sizeof(uint32_t) * experts, hipMemcpyDeviceToHost, ctx->stream);
    }
    if (err == hipSuccess) {
        err = hipStreamSynchronize(ctx->stream);
    }
    if (err != hipSuccess) {
        ttl_mxfp4_free(ctx, t);
        *out = nullptr;
        return ttl::hip_fail(err, "ttl_mxfp4_upload_dev: repack_kernel");
    }
    t->edge_experts.resize(experts);
    t->f16_inexact_experts.resize(experts);
    for (uint32_t e = 0; e < experts; ++e) {
        t->edge_experts[e] = uint8_t(edge[e] & 1u);
        t->f16_inexact_experts[e] = uint8_t((edge[e] >> 1) & 1u);
    }
    return TTL_OK;
}

int ttl_mxfp4_upload(ttl_ctx *ctx, const void *gguf_blocks, uint32_t rows, uint32_t cols, uint32_t experts,
                     ttl_mxfp4 **out) {
    TTL_REQUIRE(ctx && gguf_blocks && out, TTL_ERR_INVALID, "ttl_mxfp4_upload: null argument");
    TTL_REQUIRE(cols == uint32_t(mx::cols), TTL_ERR_SHAPE, "ttl_mxfp4_upload: cols must be %d", mx::cols);
    const size_t bytes = size_t(rows) * mx::blocks * 17 * experts;
    void *staging = nullptr;
    TTL_HIP(hipMalloc(&staging, bytes ? bytes : 1));
    int rc = ttl_memcpy_h2d(ctx, staging, gguf_blocks, bytes);
    if (rc == TTL_OK) {
        rc = ttl_mxfp4_upload_dev(ctx, staging, rows, cols, experts, out);
    }
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(staging);
    return rc;
}

int ttl_mxfp4_synthetic(ttl_ctx *ctx, uint32_t rows, uint32_t cols, uint32_t experts, uint64_t seed,
                        uint64_t stream, uint32_t emin, uint32_t emax, ttl_mxfp4 **out) {
    TTL_REQUIRE(emin <= emax && emax <= 255, TTL_ERR_INVALID, "ttl_mxfp4_synthetic: bad exponent range");
    int rc = alloc_tensor(ctx, rows, cols, experts, out, "ttl_mxfp4_synthetic");
    if (rc != TTL_OK) {
        return rc;
    }
    // every expert then holds such blocks (a block of 32 zero codes has odds 2^-128)
    (*out)->edge_experts.assign(experts, emin == 0 || emax == 255 ? 1 : 0);
    (*out)->f16_inexact_experts.assign(experts, emin < mf::f16_scale_min || emax > mf::f16_scale_max ? 1 : 0);
    return ttl::synth_mxfp4_repacked(ctx, *out, seed, stream, emin, emax);
}

int ttl_mxfp4_edge_scales(const ttl_mxfp4 *t) {
    TTL_REQUIRE(t, TTL_ERR_INVALID, "ttl_mxfp4_edge_scales: null tensor");
    return t->edge_scales() ? 1 : 0;
}

int ttl_mxfp4_f16_exact(const ttl_mxfp4 *t) {
    TTL_REQUIRE(t, TTL_ERR_INVALID, "ttl_mxfp4_f16_exact: null tensor");
    return t->f16_exact() ? 1 : 0;
}

int ttl_mxfp4_download(ttl_ctx *ctx, const ttl_mxfp4 *t, void *gguf_blocks) {
    TTL_REQUIRE(ctx && gguf_blocks, TTL_ERR_INVALID, "ttl_mxfp4_download: null argument");
    int rc = check_tensor(t, "ttl_mxfp4_download");
    if (rc != TTL_OK) {
        return rc;
    }
    const size_t n = size_t(t->rows) * mx::blocks * t->experts;
    void *staging = nullptr;
    TTL_HIP(hipMalloc(&staging, n * 17));
    unpack_kernel<<<ttl::blocks_for(n, 256), 256, 0, ctx->stream>>>((const uint4 *)t->codes, t->scales, t->rows,
                                                                     t->experts, (uint8_t *)staging);
    hipError_t err = hipGetLastError();
    rc = err == hipSuccess ? ttl_memcpy_d2h(ctx, gguf_blocks, staging, n * 17) : ttl::hip_fail(err, "unpack_kernel");
    (void)hipFree(staging);
    return rc;
}

void ttl_mxfp4_free(ttl_ctx *ctx, ttl_mxfp4 *t) {
    if (!t) {
        return;
    }
    if (ctx) {
        (void)hipStreamSynchronize(ctx->stream);
    }
    (void)hipFree(t->codes);
    (void)hipFree(t->scales);
    delete t;
}

int ttl_mxfp4_shape(const ttl_mxfp4 *t, uint32_t *rows, uint32_t *cols, uint32_t *experts) {
    TTL_REQUIRE(t, TTL_ERR_INVALID, "ttl_mxfp4_shape: null tensor");
    if (rows) {
        *rows = t->rows;
    }
    if (cols) {
        *cols = t->cols;
    }
    if (experts) {
        *experts = t->experts;
    }
    return TTL_OK;
}

size_t ttl_mxfp4_bytes(const ttl_mxfp4 *t) {
    return t ? t->code_bytes + t->scale_bytes : 0;
}

int ttl_mxfp4_dequantize(ttl_ctx *ctx, const ttl_mxfp4 *t, uint32_t expert, int mode, float *out_dev) {
    TTL_REQUIRE(ctx && out_dev, TTL_ERR_INVALID, "ttl_mxfp4_dequantize: null argument");
    int rc = check_tensor(t, "ttl_mxfp4_dequantize");
    if (rc != TTL_OK) {
        return rc;
    }
    TTL_REQUIRE(expert < t->experts, TTL_ERR_INVALID, "ttl_mxfp4_dequantize: expert %u out of range", expert);
    TTL_REQUIRE(mode >= 0 && mode <= 2, TTL_ERR_INVALID, "ttl_mxfp4_dequantize: mode must be 0, 1 or 2");
    const size_t n = size_t(t->rows) * mx::blocks;
    dequant_kernel<<<ttl::blocks_for(n, 256), 256, 0, ctx->stream>>>((const uint4 *)t->codes, t->scales, t->rows,
                                                                      expert, mode, out_dev);
    TTL_LAUNCHED("dequant_kernel");
    return TTL_OK;
}

int ttl_matvec_mxfp4_experts(ttl_ctx *ctx, const ttl_mxfp4 *w, const float *bias_dev, const float *x_dev,
                             uint32_t x_stride, const int32_t *experts_dev, uint32_t n, float *y_dev) {
    TTL_REQUIRE(ctx && x_dev && experts_dev && y_dev, TTL_ERR_INVALID, "ttl_matvec_mxfp4_experts: null argument");
    int rc = check_tensor(w, "ttl_matvec_mxfp4_experts");
    if (rc != TTL_OK) {
        return rc;
    }
    TTL_REQUIRE(x_stride == 0 || x_stride >= w->cols, TTL_ERR_SHAPE,
                "ttl_matvec_mxfp4_experts: x_stride %u smaller than cols %u", x_stride, w->cols);
    TTL_REQUIRE(x_stride % 4 == 0, TTL_ERR_SHAPE, "ttl_matvec_mxfp4_experts: x_stride must be a multiple of 4");
    TTL_REQUIRE((reinterpret_cast<uintptr_t>(x_dev) & 15) == 0, TTL_ERR_INVALID,
                "ttl_matvec_mxfp4_experts: x must be 16-byte aligned");
    if (n == 0) {
        return TTL_OK;
    }
    const size_t grid = size_t(w->tiles) * n;
    TTL_REQUIRE(grid < (1u << 31), TTL_ERR_SHAPE, "ttl_matvec_mxfp4_experts: too many slots");
    matvec_kernel<<<unsigned(grid), kMvSplit * 64, 0, ctx->stream>>>(w->codes, w->scales, w->rows, w->tiles,
                                                                     w->experts, bias_dev, x_dev, x_stride,
                                                                     experts_dev, 0u, y_dev);
    TTL_LAUNCHED("matvec_kernel");
    return TTL_OK;
}

int ttl_matvec_mxfp4(ttl_ctx *ctx, const ttl_mxfp4 *w, const float *bias_dev, const float *x_dev, float *y_dev,
                     uint32_t expert) {
    TTL_REQUIRE(ctx && x_dev && y_dev, TTL_ERR_INVALID, "ttl_matvec_mxfp4: null argument");
    int rc = check_tensor(w, "ttl_matvec_mxfp4");
    if (rc != TTL_OK) {
        return rc;
    }
    TTL_REQUIRE(expert < w->experts, TTL_ERR_INVALID, "ttl_matvec_mxfp4: expert %u out of range (%u experts)", expert,
                w->experts);
    TTL_REQUIRE((reinterpret_cast<uintptr_t>(x_dev) & 15) == 0, TTL_ERR_INVALID,
                "ttl_matvec_mxfp4: x must be 16-byte aligned");
    // the expert is known here: the kernel takes it as an argument, with no id load
    matvec_kernel<<<w->tiles, kMvSplit * 64, 0, ctx->stream>>>(w->codes, w->scales, w->rows, w->tiles, w->experts,
                                                               bias_dev, x_dev, 0u, nullptr, expert, y_dev);
    TTL_LAUNCHED("matvec_kernel");
    return TTL_OK;
}

}  // extern "C"
