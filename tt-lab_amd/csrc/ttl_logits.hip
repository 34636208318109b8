// Token embedding (load_token_embedding_q8_0, tensor.cpp:171-184), the bf16
// unembedding matvec with a per-workgroup argmax, and the greedy choice
// (GptOssModel::greedy, model.cpp:604-612).  Token and position live in device
// memory so a captured decode step can feed its own output back.
#include <hip/hip_fp16.h>

#include "ttl_internal.hpp"
#include "ttl_q8_tile.hpp"
#include "ttl_stage.hpp"

#include <cmath>

namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerWave = 4;                   // 16 lanes per row
constexpr int kRowsPerGroup = 4 * kRowsPerWave;   // 16 rows per workgroup
constexpr int kCols = 2880;
constexpr int kChunks = kCols / 8;                // 16-byte chunks of 8 bf16 per row
constexpr int kIters = (kChunks + 15) / 16;       // 23
constexpr int kXBlocks = kCols / 32;
constexpr int kMaxPartials = 1024;  // logits workgroups (4 per CU)

struct Best {
    float value;
    int32_t index;
    int32_t first_is_nan;  // set by the group holding row 0
    int32_t pad;
};

// model.cpp:604-612 as a reduction: the first index holding the largest non-NaN
// value (NaN never wins a strict '>').
__device__ inline bool better(float v, int32_t i, float bv, int32_t bi) {
    if (isnan(v)) {
        return false;
    }
    if (isnan(bv)) {
        return true;
    }
    return v > bv || (v == bv && i < bi);
}

// One workgroup stages the input once (combine + output norm fused), then walks
// row groups g = blockIdx.x, blockIdx.x + gridDim.x, ...; each wave takes 4 rows
// of a group, 16 lanes per row.  The workgroup's best (value, index) goes to
// partial[blockIdx.x].
template <int MODE>
__global__ __launch_bounds__(kThreads) void logits_kernel(const uint16_t *__restrict__ w, uint32_t rows,
                                                          stage::Input in, float *__restrict__ logits,
                                                          Best *__restrict__ partial) {
    __shared__ __attribute__((aligned(16))) float xs[kXBlocks * stage::x_stride];
    __shared__ float red[stage::red_floats(kXBlocks)];
    __shared__ float bvals[kThreads / 16];
    __shared__ int32_t bidx[kThreads / 16];
    __shared__ int32_t row0_nan;
    const uint32_t wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const uint32_t j = lane % 16;
    const uint32_t groups = (rows + kRowsPerGroup - 1) / kRowsPerGroup;
    if (blockIdx.x != 0) {
        in.v_out = nullptr;
    }
    // unconditional loads of group g's rows (a row past the end re-reads the last row)
    uint4 q[kIters];
    auto load_group = [&](uint32_t g) __attribute__((always_inline)) {
        const uint32_t row = g * kRowsPerGroup + wave * kRowsPerWave + lane / 16;
        const uint4 *src = reinterpret_cast<const uint4 *>(w + size_t(row < rows ? row : rows - 1) * kCols);
#pragma unroll
        for (int i = 0; i < kIters; ++i) {
            const uint32_t c = j + 16 * i;
            q[i] = ttl::load_stream(src + (c < uint32_t(kChunks) ? c : uint32_t(kChunks) - 1));
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // the input's loads, then the first group's weight loads, which stream while the
    // staging (the last layer's combine and the output norm) completes
    stage::Pending<kCols, kXBlocks, kThreads, MODE> pending;
    stage::stage_load(in, pending);
    load_group(blockIdx.x < groups ? blockIdx.x : groups - 1);
    stage::stage_finish(in, pending, xs, red);
    float bv = NAN;
    int32_t bi = 0x7fffffff;
    if (threadIdx.x == 0) {
        row0_nan = 0;
    }
    for (uint32_t g = blockIdx.x; g < groups; g += gridDim.x) {
        const uint32_t row = g * kRowsPerGroup + wave * kRowsPerWave + lane / 16;
        const bool valid = row < rows;
        if (g != blockIdx.x) {
            load_group(g);
        }
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < kIters; ++i) {
            const uint32_t c = j + 16 * i;
            if (c < uint32_t(kChunks)) {
                const float *xb = xs + (c / 4) * stage::x_stride + (c % 4) * 8;
                const float4 x0 = *reinterpret_cast<const float4 *>(xb);
                const float4 x1 = *reinterpret_cast<const float4 *>(xb + 4);
                const uint32_t ww[4] = {q[i].x, q[i].y, q[i].z, q[i].w};
                acc = fmaf(__uint_as_float(ww[0] << 16), x0.x, acc);
                acc = fmaf(__uint_as_float(ww[0] & 0xffff0000u), x0.y, acc);
                acc = fmaf(__uint_as_float(ww[1] << 16), x0.z, acc);
                acc = fmaf(__uint_as_float(ww[1] & 0xffff0000u), x0.w, acc);
                acc = fmaf(__uint_as_float(ww[2] << 16), x1.x, acc);
                acc = fmaf(__uint_as_float(ww[2] & 0xffff0000u), x1.y, acc);
                acc = fmaf(__uint_as_float(ww[3] << 16), x1.z, acc);
                acc = fmaf(__uint_as_float(ww[3] & 0xffff0000u), x1.w, acc);
            }
        }
#pragma unroll
        for (int d = 8; d >= 1; d >>= 1) {
            acc += __shfl_xor(acc, d);
        }
        if (j == 0 && valid) {
            logits[row] = acc;
            // rows arrive in increasing order, so better() keeps the first maximum
            if (better(acc, int32_t(row), bv, bi)) {
                bv = acc;
                bi = int32_t(row);
            }
            if (row == 0 && isnan(acc)) {
                row0_nan = 1;
            }
        }
    }
    if (j == 0) {
        bvals[threadIdx.x / 16] = bv;
        bidx[threadIdx.x / 16] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        Best b{NAN, 0x7fffffff, row0_nan, 0};
        for (int r = 0; r < kThreads / 16; ++r) {
            if (better(bvals[r], bidx[r], b.value, b.index)) {
                b.value = bvals[r];
                b.index = bidx[r];
            }
        }
        partial[blockIdx.x] = b;
    }
}

// The Q8_0 unembedding of a GGUF model (output.weight, model.cpp:598-599 through
// matvec_q8_0, tensor.cpp:202-218), with the same per-workgroup argmax as
// logits_kernel.  Rows are repacked Q8_0 tiles of 16 (ttl_q8_tile.hpp); one
// workgroup stages the input once and walks tiles blockIdx.x, blockIdx.x + gridDim.x,
// ..., the next tile's codes in flight while the current one is reduced.
template <int MODE>
__global__ __launch_bounds__(kThreads) void logits_q8_kernel(const uint8_t *__restrict__ codes,
                                                             const uint16_t *__restrict__ scales, uint32_t rows,
                                                             stage::Input in, float *__restrict__ logits,
                                                             Best *__restrict__ partial) {
    using S = q8::Shape<kCols>;
    __shared__ __attribute__((aligned(16))) float xs[S::x_blocks * stage::x_stride];
    __shared__ float xsum[S::x_blocks];
    __shared__ float red[stage::red_floats(S::x_blocks)];
    __shared__ float part[q8::waves][q8::tile_rows];
    __shared__ float bvals[q8::tile_rows];
    __shared__ int32_t bidx[q8::tile_rows];
    __shared__ int32_t row0_nan;
    const uint32_t wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const uint32_t tiles = rows / q8::tile_rows, stride = gridDim.x;
    if (blockIdx.x != 0) {
        in.v_out = nullptr;
    }
    stage::Pending<kCols, S::x_blocks, kThreads, MODE> pending;
    stage::stage_load(in, pending);
    q8::TileRegs<kCols> regs[2];
    q8::tile_load<kCols>(codes, scales, blockIdx.x, wave, lane, regs[0]);
    stage::stage_finish(in, pending, xs, red);
    q8::block_sums(xs, S::x_blocks, xsum);
    if (threadIdx.x == 0) {
        row0_nan = 0;
    }
    float bv = NAN;
    int32_t bi = 0x7fffffff;
    auto finish = [&](uint32_t t, const q8::TileRegs<kCols> &r) __attribute__((always_inline)) {
        const float acc = q8::tile_compute<kCols>(r, wave, lane, xs, xsum);
        if (lane < q8::tile_rows) {
            part[wave][lane] = acc;
        }
        __syncthreads();
        if (threadIdx.x < q8::tile_rows) {
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < q8::waves; ++w) {
                sum += part[w][threadIdx.x];
            }
            const uint32_t row = t * q8::tile_rows + threadIdx.x;
            logits[row] = sum;
            // a thread's rows arrive in increasing order, so better() keeps the first maximum
            if (better(sum, int32_t(row), bv, bi)) {
                bv = sum;
                bi = int32_t(row);
            }
            if (row == 0 && isnan(sum)) {
                row0_nan = 1;
            }
        }
        __syncthreads();
    };
    // two register sets with static indices: tile t computes while t + stride loads
    for (uint32_t t = blockIdx.x; t < tiles; t += 2 * stride) {
        const uint32_t t1 = t + stride;
        q8::tile_load<kCols>(codes, scales, min(t1, tiles - 1), wave, lane, regs[1]);
        finish(t, regs[0]);
        if (t1 >= tiles) {
            break;
        }
        q8::tile_load<kCols>(codes, scales, min(t1 + stride, tiles - 1), wave, lane, regs[0]);
        finish(t1, regs[1]);
    }
    if (threadIdx.x < q8::tile_rows) {
        bvals[threadIdx.x] = bv;
        bidx[threadIdx.x] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        Best b{NAN, 0x7fffffff, row0_nan, 0};
        for (int r = 0; r < q8::tile_rows; ++r) {
            if (better(bvals[r], bidx[r], b.value, b.index)) {
                b.value = bvals[r];
                b.index = bidx[r];
            }
        }
        partial[blockIdx.x] = b;
    }
}

// Reduces the per-group bests, writes the greedy token and advances the position.
__global__ __launch_bounds__(kThreads) void argmax_kernel(const Best *__restrict__ partial, uint32_t groups,
                                                          int32_t *__restrict__ token, int32_t *__restrict__ position,
                                                          int32_t advance, int32_t *__restrict__ history,
                                                          uint32_t history_len) {
    __shared__ float sv[kThreads];
    __shared__ int32_t si[kThreads];
    float bv = NAN;
    int32_t bi = 0x7fffffff;
    // groups <= kMaxPartials: all of a thread's loads are issued before any compare
    constexpr int kPer = (kMaxPartials + kThreads - 1) / kThreads;
    Best b[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const uint32_t g = threadIdx.x + uint32_t(k) * kThreads;
        b[k] = partial[g < groups ? g : 0];
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const uint32_t g = threadIdx.x + uint32_t(k) * kThreads;
        if (g < groups && better(b[k].value, b[k].index, bv, bi)) {
            bv = b[k].value;
            bi = b[k].index;
        }
    }
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (uint32_t s = kThreads / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s && better(sv[threadIdx.x + s], si[threadIdx.x + s], sv[threadIdx.x], si[threadIdx.x])) {
            sv[threadIdx.x] = sv[threadIdx.x + s];
            si[threadIdx.x] = si[threadIdx.x + s];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        // logits[0] NaN: the reference's loop never moves off index 0
        const int32_t choice = partial[0].first_is_nan || si[0] == 0x7fffffff ? 0 : si[0];
        *token = choice;
        if (advance) {
            const int32_t p = *position;
            if (history && p >= 0 && uint32_t(p) < history_len) {
                history[p] = choice;
            }
            *position = p + 1;
        }
    }
}

// tensor.cpp:171-184 for the token held in device memory.
__global__ __launch_bounds__(kThreads) void embedding_kernel(const uint8_t *__restrict__ table, uint32_t vocab,
                                                             const int32_t *__restrict__ token,
                                                             float *__restrict__ out) {
#pragma clang fp contract(off)
    // workgroup y embeds token[y] into out + y * 2880 (one token: y = 0)
    const int32_t tok = token[blockIdx.y];
    out += size_t(blockIdx.y) * kCols;
    const bool ok = tok >= 0 && uint32_t(tok) < vocab;
    const uint8_t *row = table + size_t(ok ? tok : 0) * (kCols / 32) * 34;
    for (uint32_t i = threadIdx.x; i < uint32_t(kCols); i += kThreads) {
        const uint8_t *blk = row + (i / 32) * 34;
        const float d = __half2float(__ushort_as_half(uint16_t(blk[0] | (blk[1] << 8))));
        out[i] = ok ? d * float(int8_t(blk[2 + i % 32])) : __builtin_nanf("");
    }
}

}  // namespace

namespace ttl {
// Workgroups of the logits launch (each writes one partial best).
size_t logits_partials(uint32_t rows) {
    const size_t groups = (rows + kRowsPerGroup - 1) / kRowsPerGroup;
    return groups < size_t(kMaxPartials) ? groups : size_t(kMaxPartials);
}
}  // namespace ttl

extern "C" {

size_t ttl_logits_workspace_bytes(uint32_t vocab) {
    return ttl::logits_partials(vocab) * sizeof(Best);
}

int ttl_logits_bf16(ttl_ctx *ctx, const uint16_t *weight_dev, uint32_t vocab, const ttl_stage_input *in,
                    float *logits_dev, void *workspace_dev) {
    TTL_REQUIRE(ctx && weight_dev && logits_dev && workspace_dev, TTL_ERR_INVALID, "ttl_logits_bf16: null argument");
    const int rc = stage::check(in, "ttl_logits_bf16");
    if (rc != TTL_OK) {
        return rc;
    }
    TTL_REQUIRE(vocab > 0, TTL_ERR_SHAPE, "ttl_logits_bf16: vocab must be positive");
    TTL_REQUIRE(((uintptr_t)weight_dev & 15) == 0, TTL_ERR_INVALID, "ttl_logits_bf16: weights must be 16-byte aligned");
    const stage::Input s = stage::from_abi(in);
    const uint32_t groups = uint32_t(ttl::logits_partials(vocab));
    stage::with_mode(s, [&](auto mode) {
        logits_kernel<decltype(mode)::value><<<groups, kThreads, 0, ctx->stream>>>(
            weight_dev, vocab, s, logits_dev, reinterpret_cast<Best *>(workspace_dev));
    });
    TTL_LAUNCHED("logits_kernel");
    return TTL_OK;
}

int ttl_logits_q8_0(ttl_ctx *ctx, const ttl_q8 *weight, uint32_t vocab, const ttl_stage_input *in, float *logits_dev,
                    void *workspace_dev) {
    TTL_REQUIRE(ctx && weight && weight->codes && weight->scales && logits_dev && workspace_dev, TTL_ERR_INVALID,
                "ttl_logits_q8_0: null argument");
    const int rc = stage::check(in, "ttl_logits_q8_0");
    if (rc != TTL_OK) {
        return rc;
    }
    TTL_REQUIRE(weight->cols == uint32_t(kCols) && weight->rows == vocab && vocab > 0, TTL_ERR_SHAPE,
                "ttl_logits_q8_0: the tensor must be vocab x %d (got %u x %u, vocab %u)", kCols, weight->rows,
                weight->cols, vocab);
    const stage::Input s = stage::from_abi(in);
    const uint32_t groups = uint32_t(ttl::logits_partials(vocab));  // vocab / 16 tiles, at most 1024 workgroups
    stage::with_mode(s, [&](auto mode) {
        logits_q8_kernel<decltype(mode)::value><<<groups, kThreads, 0, ctx->stream>>>(
            weight->codes, weight->scales, vocab, s, logits_dev, reinterpret_cast<Best *>(workspace_dev));
    });
    TTL_LAUNCHED("logits_q8_kernel");
    return TTL_OK;
}

int ttl_argmax(ttl_ctx *ctx, uint32_t vocab, const void *workspace_dev, int32_t *token_dev, int32_t *position_dev,
               int32_t *history_dev, uint32_t history_len) {
    TTL_REQUIRE(ctx && workspace_dev && token_dev, TTL_ERR_INVALID, "ttl_argmax: null argument");
    argmax_kernel<<<1, kThreads, 0, ctx->stream>>>(reinterpret_cast<const Best *>(workspace_dev),
                                                   uint32_t(ttl::logits_partials(vocab)), token_dev,
                                                   position_dev ? position_dev : token_dev, position_dev ? 1 : 0,
                                                   history_dev, history_len);
    TTL_LAUNCHED("argmax_kernel");
    return TTL_OK;
}

int ttl_embedding_q8_0(ttl_ctx *ctx, const void *table_dev, uint32_t vocab, const int32_t *token_dev,
                       float *out_dev) {
    TTL_REQUIRE(ctx && table_dev && token_dev && out_dev, TTL_ERR_INVALID, "ttl_embedding_q8_0: null argument");
    embedding_kernel<<<1, kThreads, 0, ctx->stream>>>((const uint8_t *)table_dev, vocab, token_dev, out_dev);
    TTL_LAUNCHED("embedding_kernel");
    return TTL_OK;
}

int ttl_embedding_q8_0_batch(ttl_ctx *ctx, const void *table_dev, uint32_t vocab, const int32_t *tokens_dev,
                             uint32_t count, float *out_dev) {
    TTL_REQUIRE(ctx && table_dev && tokens_dev && out_dev, TTL_ERR_INVALID, "ttl_embedding_q8_0_batch: null argument");
    TTL_REQUIRE(count <= 65535, TTL_ERR_SHAPE, "ttl_embedding_q8_0_batch: at most 65535 tokens per call");
    if (count == 0) {
        return TTL_OK;
    }
    embedding_kernel<<<dim3(1, count), kThreads, 0, ctx->stream>>>((const uint8_t *)table_dev, vocab, tokens_dev,
                                                                   out_dev);
    TTL_LAUNCHED("embedding_kernel");
    return TTL_OK;
}

}  // extern "C"
