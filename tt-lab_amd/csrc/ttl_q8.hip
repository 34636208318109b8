// Q8_0 tensors and the attention-side matvecs of the decode step:
//   - generic y = W x (+ b)                  matvec_q8_0 / matvec_add_q8_0 (tensor.cpp:202-237)
//   - fused Q/K/V projection                 model.cpp:572-582: rms_norm, three matvec_add_q8_0,
//     (+ norm/combine prologue, RoPE,        apply_rope on q and k, store_kv
//      KV-cache store epilogue)
//   - output projection + residual add       model.cpp:584-588
#include <hip/hip_fp16.h>

#include "ttl_mfma.hpp"
#include "ttl_q8_tile.hpp"

namespace {

constexpr int kHead = 64, kQHeads = 64, kKvHeads = 8;
constexpr int kQRows = kQHeads * kHead, kKvRows = kKvHeads * kHead, kQkvRows = kQRows + 2 * kKvRows;

// ---- layout conversion ---------------------------------------------------------

__global__ void q8_repack_kernel(const uint8_t *__restrict__ gguf, uint32_t rows, uint32_t cols,
                                 const int32_t *__restrict__ row_source, uint8_t *__restrict__ codes,
                                 uint16_t *__restrict__ scales, uint16_t *__restrict__ row_scales) {
    const uint32_t blocks = cols / 32;
    const size_t gid = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= size_t(rows) * blocks) {
        return;
    }
    const uint32_t row = uint32_t(gid / blocks), block = uint32_t(gid % blocks);
    const uint32_t src_row = row_source ? uint32_t(row_source[row]) : row;
    const uint8_t *src = gguf + (size_t(src_row) * blocks + block) * 34;
    const size_t tile = row / q8::tile_rows;
    const uint32_t r = row % q8::tile_rows;
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        w[i] = uint32_t(src[2 + 4 * i]) | (uint32_t(src[3 + 4 * i]) << 8) | (uint32_t(src[4 + 4 * i]) << 16) |
               (uint32_t(src[5 + 4 * i]) << 24);
    }
    *reinterpret_cast<uint4 *>(codes + q8::code_offset(tile, block, 0, r, int(cols))) = make_uint4(w[0], w[1], w[2], w[3]);
    *reinterpret_cast<uint4 *>(codes + q8::code_offset(tile, block, 1, r, int(cols))) = make_uint4(w[4], w[5], w[6], w[7]);
    const uint16_t d = uint16_t(src[0] | (src[1] << 8));
    scales[q8::scale_index(tile, block, r, int(cols))] = d;
    row_scales[size_t(row) * q8::row_scale_stride(int(cols)) + block] = d;
}

__global__ void q8_unpack_kernel(const uint8_t *__restrict__ codes, const uint16_t *__restrict__ scales,
                                 uint32_t rows, uint32_t cols, uint8_t *__restrict__ gguf) {
    const uint32_t blocks = cols / 32;
    const size_t gid = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= size_t(rows) * blocks) {
        return;
    }
    const uint32_t row = uint32_t(gid / blocks), block = uint32_t(gid % blocks);
    const size_t tile = row / q8::tile_rows;
    const uint32_t r = row % q8::tile_rows;
    const uint16_t s = scales[q8::scale_index(tile, block, r, int(cols))];
    uint8_t *dst = gguf + gid * 34;
    dst[0] = uint8_t(s);
    dst[1] = uint8_t(s >> 8);
    for (uint32_t h = 0; h < 2; ++h) {
        const uint8_t *src = codes + q8::code_offset(tile, block, h, r, int(cols));
        for (int i = 0; i < 16; ++i) {
            dst[2 + 16 * h + i] = src[i];
        }
    }
}

// GGUF Q8_0 blocks from the synthetic generator (same bits as oracle orc_synth_q8_0).
__global__ void q8_synth_kernel(uint64_t seed, uint64_t stream, size_t block_offset, size_t n, uint8_t *out) {
    const size_t k = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (k >= n) {
        return;
    }
    const uint64_t b = block_offset + k;
    uint8_t *dst = out + k * 34;
    const uint32_t scale = 0x0c00u | uint32_t(synth::hash(seed, stream, 5 * b) & 0x3ffu);
    dst[0] = uint8_t(scale);
    dst[1] = uint8_t(scale >> 8);
    for (int w = 0; w < 4; ++w) {
        const uint64_t h = synth::hash(seed, stream, 5 * b + 1 + uint64_t(w));
        for (int i = 0; i < 8; ++i) {
            dst[2 + 8 * w + i] = uint8_t(h >> (8 * i));
        }
    }
}

// ---- matvec kernels -------------------------------------------------------------

struct NoLoads {
    __device__ void operator()() const {}
};

// Common body: one workgroup = one 16-row tile; returns the row sum for row
// threadIdx.x (valid for threadIdx.x < 16) after the wave-order reduction.
// late_loads() runs once the input and weight loads are issued: loads whose
// addresses wait on another load (the qkv epilogue's RoPE pair waits on the
// position) go there, so that wait does not hold back the weight stream.
template <int K, int W, int MODE, class LateLoads = NoLoads>
__device__ __attribute__((always_inline)) inline float tile_matvec(const uint8_t *__restrict__ codes,
                                                                  const uint16_t *__restrict__ scales,
                                                                  size_t tile, const stage::Input &in,
                                                                  float *xs, float *xsum, float *red,
                                                                  float (*part)[q8::tile_rows],
                                                                  LateLoads &&late_loads = NoLoads{}) {
    using S = q8::Shape<K>;
    const uint32_t wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    // input loads first: the staging then waits for them alone while the weight
    // loads are still in flight
    stage::Pending<K, S::x_blocks, W * 64, MODE> pending;
    stage::stage_load(in, pending);
    q8::TileRegs<K, W> regs;
    q8::tile_load<K, W>(codes, scales, tile, wave, lane, regs);
    late_loads();
    stage::stage_finish(in, pending, xs, red);
    q8::block_sums(xs, S::x_blocks, xsum);
    const float acc = q8::tile_compute<K, W>(regs, wave, lane, xs, xsum);
    if (lane < q8::tile_rows) {
        part[wave][lane] = acc;
    }
    __syncthreads();
    float sum = 0.0f;
    if (threadIdx.x < q8::tile_rows) {
#pragma unroll
        for (int w = 0; w < W; ++w) {
            sum += part[w][threadIdx.x];
        }
    }
    return sum;
}

// Waves per tile (each divides its K's padded iterations, 24 and 32): measured on
// the decode step, 12 and 8 beat 4 (the layout's own split), 6 and 16.  More waves
// shorten each wave's decode chain after its loads arrive.
template <int K>
constexpr int waves_for() {
    return K == 2880 ? 12 : 8;
}

template <int K, int MODE>
__global__ __launch_bounds__(waves_for<K>() * 64) void q8_matvec_kernel(const uint8_t *__restrict__ codes,
                                                                        const uint16_t *__restrict__ scales,
                                                                        uint32_t rows, stage::Input in,
                                                                        const float *__restrict__ bias,
                                                                        const float *__restrict__ residual,
                                                                        float *__restrict__ y) {
    constexpr int W = waves_for<K>();
    __shared__ __attribute__((aligned(16))) float xs[q8::Shape<K>::x_blocks * stage::x_stride];
    __shared__ float xsum[q8::Shape<K>::x_blocks];
    __shared__ float red[stage::red_floats(q8::Shape<K>::x_blocks)];
    __shared__ float part[W][q8::tile_rows];
    const size_t tile = blockIdx.x;
    if (blockIdx.x != 0) {
        in.v_out = nullptr;
    }
    // epilogue operands first, so no load waits at the end (rows is a multiple of 16)
    const uint32_t row = uint32_t(tile) * q8::tile_rows + threadIdx.x % q8::tile_rows;
    const float bv = bias ? bias[row] : 0.0f;
    const float rv = residual ? residual[row] : 0.0f;
    const float sum = tile_matvec<K, W, MODE>(codes, scales, tile, in, xs, xsum, red, part);
    if (threadIdx.x < q8::tile_rows) {
        // tensor.cpp:235: bias + sum; model.cpp:586-588: residual = x + projected
        const float projected = bias ? bv + sum : sum;
        y[row] = residual ? rv + projected : projected;
    }
}

// Q/K/V rows repacked as 320 tiles: q heads (tiles 0..255), k heads (256..287),
// v heads (288..319), four tiles per head.  In q and k tiles, tile j of a head holds
// dims 8j..8j+7 (lanes 0..7) and 32+8j..32+8j+7 (lanes 8..15), so the RoPE pairs
// (d, d+32) of model.cpp:235-243 meet in lanes (r, r+8); v tiles hold dims 16j..16j+15.
__host__ __device__ inline uint32_t qkv_dim(uint32_t tile, uint32_t r) {
    const uint32_t j = tile % 4;
    if (tile >= uint32_t(kQHeads + kKvHeads) * 4) {
        return 16 * j + r;
    }
    return r < 8 ? 8 * j + r : 32 + 8 * j + (r - 8);
}

template <int MODE>
__global__ __launch_bounds__(waves_for<2880>() * 64) void qkv_kernel(const uint8_t *__restrict__ codes,
                                                       const uint16_t *__restrict__ scales, stage::Input in,
                                                       const float *__restrict__ bias,
                                                       const float2 *__restrict__ rope,
                                                       const int32_t *__restrict__ position,
                                                       uint32_t capacity, float *__restrict__ q_out,
                                                       float *__restrict__ k_cache, float *__restrict__ v_cache) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float xs[q8::Shape<2880>::x_blocks * stage::x_stride];
    __shared__ float xsum[q8::Shape<2880>::x_blocks];
    __shared__ float red[stage::red_floats(q8::Shape<2880>::x_blocks)];
    constexpr int W = waves_for<2880>();
    __shared__ float part[W][q8::tile_rows];
    __shared__ float vals[q8::tile_rows];
    const uint32_t tile = blockIdx.x;
    if (blockIdx.x != 0) {
        in.v_out = nullptr;
    }
    // epilogue operands before the sum, so no load waits at the end: the bias first;
    // the position and the RoPE pair it selects once the weight loads are issued
    const uint32_t r = threadIdx.x, r16 = r % q8::tile_rows;
    const bool is_q = tile < uint32_t(kQHeads) * 4, is_k = !is_q && tile < uint32_t(kQHeads + kKvHeads) * 4;
    const uint32_t head = is_q ? tile / 4 : (is_k ? (tile - kQHeads * 4) / 4 : (tile - (kQHeads + kKvHeads) * 4) / 4);
    const uint32_t base = is_q ? 0u : (is_k ? uint32_t(kQRows) : uint32_t(kQRows + kKvRows));
    const uint32_t dim = qkv_dim(tile, r16);
    const float bv = bias[base + head * kHead + dim];
    const uint32_t pair = (r16 < 8 ? dim : dim - 32) % 32;  // v rows: any in-bounds pair, unused
    uint32_t pos = 0;
    float2 cs;
    const float sum = tile_matvec<2880, W, MODE>(codes, scales, tile, in, xs, xsum, red, part, [&]() {
        // unconditional (a clamped position), so the compiler need not wait for every
        // load in flight at the end of a branch
        pos = uint32_t(*position);
        cs = rope[size_t(min(pos, capacity - 1)) * (kHead / 2) + pair];
    });
    if (r < q8::tile_rows) {
        vals[r] = bv + sum;
    }
    __syncthreads();
    if (r >= q8::tile_rows || pos >= capacity) {
        return;
    }
    float out = vals[r];
    if (!(is_q || is_k)) {
        v_cache[(size_t(pos) * kKvHeads + head) * kHead + dim] = out;
        return;
    }
    // model.cpp:236-242 with cos/sin precomputed by the host exactly as the reference does
    const float x = vals[r < 8 ? r : r - 8];
    const float yv = vals[r < 8 ? r + 8 : r];
    out = r < 8 ? x * cs.x - yv * cs.y : x * cs.y + yv * cs.x;
    if (is_q) {
        q_out[head * kHead + dim] = out;
    } else {
        k_cache[(size_t(pos) * kKvHeads + head) * kHead + dim] = out;
    }
}

// ---- batched prefill helpers -------------------------------------------------------

// Bias, RoPE and the KV-cache store of a batch of tokens (model.cpp:499-507) from the
// batched Q/K/V matmul (rows in ttl_qkv_row_source order, no bias): token t sits at
// position first + t.  One thread per (row, token); a q/k row's RoPE partner is row
// r ^ 8 of the same tile.  The rotation is qkv_kernel's, unfused.
__global__ __launch_bounds__(256) void qkv_rope_store_kernel(const float *__restrict__ qkv, uint32_t first,
                                                             const float *__restrict__ bias,
                                                             const float2 *__restrict__ rope,
                                                             float *__restrict__ q_out, float *__restrict__ k_cache,
                                                             float *__restrict__ v_cache) {
#pragma clang fp contract(off)
    const uint32_t token = blockIdx.y, row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= uint32_t(kQkvRows)) {
        return;
    }
    const uint32_t tile = row / q8::tile_rows, r16 = row % q8::tile_rows;
    const bool is_q = tile < uint32_t(kQHeads) * 4, is_k = !is_q && tile < uint32_t(kQHeads + kKvHeads) * 4;
    const uint32_t head = is_q ? tile / 4 : (is_k ? (tile - kQHeads * 4) / 4 : (tile - (kQHeads + kKvHeads) * 4) / 4);
    const uint32_t base = is_q ? 0u : (is_k ? uint32_t(kQRows) : uint32_t(kQRows + kKvRows));
    const uint32_t dim = qkv_dim(tile, r16);
    const float *in = qkv + size_t(token) * kQkvRows;
    const float value = bias[base + head * kHead + dim] + in[row];
    const uint32_t pos = first + token;
    if (!(is_q || is_k)) {
        v_cache[(size_t(pos) * kKvHeads + head) * kHead + dim] = value;
        return;
    }
    const uint32_t r2 = r16 ^ 8u, dim2 = qkv_dim(tile, r2);
    const float partner = bias[base + head * kHead + dim2] + in[tile * q8::tile_rows + r2];
    const uint32_t pair = r16 < 8 ? dim : dim - 32;
    const float2 cs = rope[size_t(pos) * (kHead / 2) + pair];
    const float x = r16 < 8 ? value : partner, y = r16 < 8 ? partner : value;
    const float out = r16 < 8 ? x * cs.x - y * cs.y : x * cs.y + y * cs.x;
    if (is_q) {
        q_out[size_t(token) * kQRows + head * kHead + dim] = out;
    } else {
        k_cache[(size_t(pos) * kKvHeads + head) * kHead + dim] = out;
    }
}

// rms_norm (tensor.cpp:568-580) of row blockIdx.x of x [rows][2880], in the staging's
// canonical order (so a row normalizes to the same bits as in the decode kernels).
// shift, if not null, receives the normalized row's f16-plane shift (mf::row_shift of
// its largest finite magnitude), as ttl::launch_row_shifts would compute it.
__global__ __launch_bounds__(256) void rms_norm_rows_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                            float eps, float *__restrict__ out,
                                                            int32_t *__restrict__ shift) {
    using S = q8::Shape<2880>;
    __shared__ __attribute__((aligned(16))) float xs[S::x_blocks * stage::x_stride];
    __shared__ float red[stage::red_floats(S::x_blocks)];
    __shared__ float wave_m[4];
    stage::Input in{};
    in.base = x + size_t(blockIdx.x) * 2880;
    in.norm_w = w;
    in.eps = eps;
    stage::stage<2880, S::x_blocks, 256, stage::kNorm>(in, xs, red);
    float *o = out + size_t(blockIdx.x) * 2880;
    float m = 0.0f;
    for (uint32_t c = threadIdx.x; c < 2880u; c += 256) {
        const float v = xs[(c / 32) * stage::x_stride + c % 32];
        o[c] = v;
        m = mf::finite_max(m, v);
    }
    if (shift) {
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) {
            m = __builtin_fmaxf(m, __shfl_xor(m, d));
        }
        if (threadIdx.x % 64 == 0) {
            wave_m[threadIdx.x / 64] = m;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            const float mm = __builtin_fmaxf(__builtin_fmaxf(wave_m[0], wave_m[1]), __builtin_fmaxf(wave_m[2], wave_m[3]));
            shift[blockIdx.x] = mf::row_shift(mm);
        }
    }
}

__global__ void add_kernel(const float *__restrict__ a, const float *__restrict__ b, size_t n, float *__restrict__ out) {
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) {
        out[i] = a[i] + b[i];
    }
}

int check_q8(const ttl_q8 *t, const char *who) {
    TTL_REQUIRE(t && t->codes && t->scales, TTL_ERR_INVALID, "%s: null tensor", who);
    return TTL_OK;
}

}  // namespace

extern "C" {

int ttl_q8_upload_dev(ttl_ctx *ctx, const void *gguf_dev, uint32_t rows, uint32_t cols, const int32_t *row_source,
                      ttl_q8 **out) {
    TTL_REQUIRE(ctx && gguf_dev && out, TTL_ERR_INVALID, "ttl_q8_upload_dev: null argument");
    *out = nullptr;
    TTL_REQUIRE(cols == 2880 || cols == 4096, TTL_ERR_SHAPE, "ttl_q8_upload_dev: cols must be 2880 or 4096");
    TTL_REQUIRE(rows > 0 && rows % q8::tile_rows == 0, TTL_ERR_SHAPE, "ttl_q8_upload_dev: rows must be a multiple of 16");
    ttl_q8 *t = new ttl_q8;
    t->rows = rows;
    t->cols = cols;
    t->tiles = rows / q8::tile_rows;
    t->code_bytes = size_t(t->tiles) * q8::blocks_of(int(cols)) * q8::tile_rows * 32;
    t->scale_bytes = size_t(t->tiles) * q8::lanes_k * q8::tile_rows * q8::scale_pad_of(int(cols)) * 2;
    int32_t *perm = nullptr;
    const size_t tail = q8::tail_pad_bytes(int(cols));
    hipError_t err = hipMalloc(&t->codes, t->code_bytes + tail);
    if (err == hipSuccess) {
        err = hipMalloc(&t->scales, t->scale_bytes);
    }
    const size_t row_scale_bytes = size_t(rows) * q8::row_scale_stride(int(cols)) * sizeof(uint16_t);
    if (err == hipSuccess) {
        err = hipMalloc(&t->row_scales, row_scale_bytes);
    }
    if (err == hipSuccess) {
        err = hipMemsetAsync(t->row_scales, 0, row_scale_bytes, ctx->stream);
    }
    if (err == hipSuccess) {
        err = hipMemsetAsync(t->scales, 0, t->scale_bytes, ctx->stream);
    }
    if (err == hipSuccess && tail) {
        err = hipMemsetAsync(t->codes + t->code_bytes, 0, tail, ctx->stream);
    }
    if (err == hipSuccess && row_source) {
        err = hipMalloc(&perm, sizeof(int32_t) * rows);
        if (err == hipSuccess) {
            err = hipMemcpyAsync(perm, row_source, sizeof(int32_t) * rows, hipMemcpyHostToDevice, ctx->stream);
        }
    }
    if (err == hipSuccess) {
        const size_t n = size_t(rows) * (cols / 32);
        q8_repack_kernel<<<ttl::blocks_for(n, 256), 256, 0, ctx->stream>>>((const uint8_t *)gguf_dev, rows, cols,
                                                                            perm, t->codes, t->scales,
                                                                            t->row_scales);
        err = hipGetLastError();
    }
    if (err == hipSuccess) {
        err = hipStreamSynchronize(ctx->stream);
    }
    (void)hipFree(perm);
    if (err != hipSuccess) {
        ttl_q8_free(ctx, t);
        return ttl::hip_fail(err, "ttl_q8_upload_dev");
    }
    *out = t;
    return TTL_OK;
}

int ttl_q8_upload(ttl_ctx *ctx, const void *gguf_blocks, uint32_t rows, uint32_t cols, const int32_t *row_source,
                  uint32_t source_rows, ttl_q8 **out) {
    TTL_REQUIRE(ctx && gguf_blocks && out, TTL_ERR_INVALID, "ttl_q8_upload: null argument");
    TTL_REQUIRE(cols % 32 == 0, TTL_ERR_SHAPE, "ttl_q8_upload: cols must be a multiple of 32");
    if (row_source) {
        for (uint32_t i = 0; i < rows; ++i) {
            TTL_REQUIRE(row_source[i] >= 0 && uint32_t(row_source[i]) < source_rows, TTL_ERR_INVALID,
                        "ttl_q8_upload: row_source[%u] out of range", i);
        }
    } else {
        TTL_REQUIRE(source_rows == rows, TTL_ERR_SHAPE, "ttl_q8_upload: source_rows must equal rows");
    }
    const size_t bytes = size_t(source_rows) * (cols / 32) * 34;
    void *staging = nullptr;
    TTL_HIP(hipMalloc(&staging, bytes));
    int rc = ttl_memcpy_h2d(ctx, staging, gguf_blocks, bytes);
    if (rc == TTL_OK) {
        rc = ttl_q8_upload_dev(ctx, staging, rows, cols, row_source, out);
    }
    (void)hipFree(staging);
    return rc;
}

int ttl_q8_download(ttl_ctx *ctx, const ttl_q8 *t, void *gguf_blocks) {
    TTL_REQUIRE(ctx && gguf_blocks, TTL_ERR_INVALID, "ttl_q8_download: null argument");
    int rc = check_q8(t, "ttl_q8_download");
    if (rc != TTL_OK) {
        return rc;
    }
    const size_t n = size_t(t->rows) * (t->cols / 32);
    void *staging = nullptr;
    TTL_HIP(hipMalloc(&staging, n * 34));
    q8_unpack_kernel<<<ttl::blocks_for(n, 256), 256, 0, ctx->stream>>>(t->codes, t->scales, t->rows, t->cols,
                                                                        (uint8_t *)staging);
    const hipError_t err = hipGetLastError();
    rc = err == hipSuccess ? ttl_memcpy_d2h(ctx, gguf_blocks, staging, n * 34) : ttl::hip_fail(err, "q8_unpack");
    (void)hipFree(staging);
    return rc;
}

void ttl_q8_free(ttl_ctx *ctx, ttl_q8 *t) {
    if (!t) {
        return;
    }
    if (ctx) {
        (void)hipStreamSynchronize(ctx->stream);
    }
    (void)hipFree(t->codes);
    (void)hipFree(t->scales);
    (void)hipFree(t->row_scales);
    delete t;
}

size_t ttl_q8_bytes(const ttl_q8 *t) {
    return t ? t->code_bytes + t->scale_bytes + size_t(t->rows) * q8::row_scale_stride(int(t->cols)) * sizeof(uint16_t)
             : 0;
}

int ttl_synth_q8_0_gguf(ttl_ctx *ctx, uint64_t seed, uint64_t stream, size_t block_offset, size_t n,
                        uint8_t *out_dev) {
    TTL_REQUIRE(ctx && (n == 0 || out_dev), TTL_ERR_INVALID, "ttl_synth_q8_0_gguf: null argument");
    if (n) {
        q8_synth_kernel<<<ttl::blocks_for(n, 256), 256, 0, ctx->stream>>>(seed, stream, block_offset, n, out_dev);
        TTL_LAUNCHED("q8_synth_kernel");
    }
    return TTL_OK;
}

int ttl_qkv_row_source(int32_t *row_source) {
    TTL_REQUIRE(row_source, TTL_ERR_INVALID, "ttl_qkv_row_source: null argument");
    for (uint32_t tile = 0; tile < uint32_t(kQkvRows) / q8::tile_rows; ++tile) {
        const bool is_q = tile < uint32_t(kQHeads) * 4, is_k = !is_q && tile < uint32_t(kQHeads + kKvHeads) * 4;
        const uint32_t head =
            is_q ? tile / 4 : (is_k ? (tile - kQHeads * 4) / 4 : (tile - (kQHeads + kKvHeads) * 4) / 4);
        const uint32_t base = is_q ? 0u : (is_k ? uint32_t(kQRows) : uint32_t(kQRows + kKvRows));
        for (uint32_t r = 0; r < q8::tile_rows; ++r) {
            row_source[tile * q8::tile_rows + r] = int32_t(base + head * kHead + qkv_dim(tile, r));
        }
    }
    return TTL_OK;
}

int ttl_matvec_q8_0(ttl_ctx *ctx, const ttl_q8 *w, const float *bias_dev, const ttl_stage_input *in,
                    const float *residual_dev, float *y_dev) {
    TTL_REQUIRE(ctx && y_dev, TTL_ERR_INVALID, "ttl_matvec_q8_0: null argument");
    int rc = check_q8(w, "ttl_matvec_q8_0");
    if (rc == TTL_OK) {
        rc = stage::check(in, "ttl_matvec_q8_0");
    }
    if (rc != TTL_OK) {
        return rc;
    }
    const stage::Input s = stage::from_abi(in);
    stage::with_mode(s, [&](auto mode) {
        constexpr int M = decltype(mode)::value;
        if (w->cols == 2880) {
            q8_matvec_kernel<2880, M><<<w->tiles, waves_for<2880>() * 64, 0, ctx->stream>>>(w->codes, w->scales, w->rows, s,
                                                                             bias_dev, residual_dev, y_dev);
        } else {
            q8_matvec_kernel<4096, M><<<w->tiles, waves_for<4096>() * 64, 0, ctx->stream>>>(w->codes, w->scales, w->rows, s,
                                                                             bias_dev, residual_dev, y_dev);
        }
    });
    TTL_LAUNCHED("q8_matvec_kernel");
    return TTL_OK;
}

int ttl_attn_qkv(ttl_ctx *ctx, const ttl_q8 *qkv, const float *bias_dev, const ttl_stage_input *in,
                 const float *rope_dev, const int32_t *position_dev, uint32_t capacity, float *q_dev,
                 float *k_cache_dev, float *v_cache_dev) {
    TTL_REQUIRE(ctx && bias_dev && rope_dev && position_dev && q_dev && k_cache_dev && v_cache_dev, TTL_ERR_INVALID,
                "ttl_attn_qkv: null argument");
    int rc = check_q8(qkv, "ttl_attn_qkv");
    if (rc == TTL_OK) {
        rc = stage::check(in, "ttl_attn_qkv");
    }
    if (rc != TTL_OK) {
        return rc;
    }
    TTL_REQUIRE(qkv->rows == uint32_t(kQkvRows) && qkv->cols == 2880, TTL_ERR_SHAPE,
                "ttl_attn_qkv: the QKV tensor must be 5120 x 2880 (q|k|v rows in ttl_qkv_row_source order)");
    const stage::Input s = stage::from_abi(in);
    stage::with_mode(s, [&](auto mode) {
        qkv_kernel<decltype(mode)::value><<<qkv->tiles, waves_for<2880>() * 64, 0, ctx->stream>>>(
            qkv->codes, qkv->scales, s, bias_dev, reinterpret_cast<const float2 *>(rope_dev), position_dev, capacity,
            q_dev, k_cache_dev, v_cache_dev);
    });
    TTL_LAUNCHED("qkv_kernel");
    return TTL_OK;
}

int ttl_qkv_rope_store(ttl_ctx *ctx, const float *qkv_dev, uint32_t tokens, uint32_t first_position,
                       const float *bias_dev, const float *rope_dev, uint32_t capacity, float *q_dev,
                       float *k_cache_dev, float *v_cache_dev) {
    TTL_REQUIRE(ctx && qkv_dev && bias_dev && rope_dev && q_dev && k_cache_dev && v_cache_dev, TTL_ERR_INVALID,
                "ttl_qkv_rope_store: null argument");
    TTL_REQUIRE(tokens <= 65535 && size_t(first_position) + tokens <= capacity, TTL_ERR_SHAPE,
                "ttl_qkv_rope_store: positions past the capacity %u", capacity);
    if (tokens == 0) {
        return TTL_OK;
    }
    qkv_rope_store_kernel<<<dim3(kQkvRows / 256, tokens), 256, 0, ctx->stream>>>(
        qkv_dev, first_position, bias_dev, reinterpret_cast<const float2 *>(rope_dev), q_dev, k_cache_dev, v_cache_dev);
    TTL_LAUNCHED("qkv_rope_store_kernel");
    return TTL_OK;
}

int ttl_rms_norm_rows_shifts(ttl_ctx *ctx, const float *x_dev, uint32_t rows, const float *weight_dev,
                             float epsilon, float *out_dev, int32_t *shift_dev) {
    TTL_REQUIRE(ctx && x_dev && weight_dev && out_dev, TTL_ERR_INVALID, "ttl_rms_norm_rows: null argument");
    TTL_REQUIRE(((uintptr_t)x_dev & 15) == 0 && ((uintptr_t)weight_dev & 15) == 0, TTL_ERR_INVALID,
                "ttl_rms_norm_rows: x and weight must be 16-byte aligned");
    TTL_REQUIRE(rows < (1u << 31), TTL_ERR_SHAPE, "ttl_rms_norm_rows: too many rows");
    if (rows == 0) {
        return TTL_OK;
    }
    rms_norm_rows_kernel<<<rows, 256, 0, ctx->stream>>>(x_dev, weight_dev, epsilon, out_dev, shift_dev);
    TTL_LAUNCHED("rms_norm_rows_kernel");
    return TTL_OK;
}

int ttl_rms_norm_rows(ttl_ctx *ctx, const float *x_dev, uint32_t rows, const float *weight_dev, float epsilon,
                      float *out_dev) {
    return ttl_rms_norm_rows_shifts(ctx, x_dev, rows, weight_dev, epsilon, out_dev, nullptr);
}

int ttl_add(ttl_ctx *ctx, const float *a_dev, const float *b_dev, size_t n, float *out_dev) {
    TTL_REQUIRE(ctx && a_dev && b_dev && out_dev, TTL_ERR_INVALID, "ttl_add: null argument");
    if (n == 0) {
        return TTL_OK;
    }
    add_kernel<<<ttl::blocks_for(n, 256), 256, 0, ctx->stream>>>(a_dev, b_dev, n, out_dev);
    TTL_LAUNCHED("add_kernel");
    return TTL_OK;
}

}  // extern "C"
