// Context, errors, device memory and timing entry points of the C ABI.
#include "ttl_internal.hpp"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>

namespace {
thread_local char last_error[512] = "";

__global__ void fill_bytes_kernel(uint8_t *dst, uint8_t value, size_t n) {
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t k = i; k < n; k += stride) {
        dst[k] = value;
    }
}

// 16-byte vector copy, grid-stride: the known-size reference dispatch for the byte
// counters (each byte read once and written once).
__global__ void copy16_kernel(const uint4 *__restrict__ src, uint4 *__restrict__ dst, size_t n) {
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t k = i; k < n; k += stride) {
        dst[k] = src[k];
    }
}

// Plain streaming read, the bandwidth reference for the matvec kernels: a grid of at
// most kReadBlocks workgroups strides over the words, each thread keeping four 16-byte
// loads in flight per pass, marked non-temporal like the weight loads of the kernels it
// is the reference for (ttl::load_stream).  Measured at 35.4 MB per launch (24 buffers
// in a graph, ordinary loads): 6.96 us with 512 or 1024 workgroups, against 7.33 us for
// one pass of 4 loads per thread over 2160 workgroups and 7.4-8.5 us for 8 or 16 loads
// per thread or 256 workgroups.  The XOR of the words is stored only when it equals a
// fixed constant, so the loads stay live and nothing is written in practice.
constexpr int kReadThreads = 256, kReadPerThread = 4, kReadBlocks = 1024;
__global__ __launch_bounds__(kReadThreads) void stream_read_kernel(const uint4 *__restrict__ src, size_t n,
                                                                   uint32_t *__restrict__ sink) {
    const size_t stride = size_t(gridDim.x) * kReadThreads * kReadPerThread;
    uint32_t acc = 0;
    for (size_t base = size_t(blockIdx.x) * kReadThreads * kReadPerThread + threadIdx.x; base < n; base += stride) {
        uint4 v[kReadPerThread];
#pragma unroll
        for (int k = 0; k < kReadPerThread; ++k) {
            const size_t i = base + size_t(k) * kReadThreads;
            v[k] = ttl::load_stream(src + (i < n ? i : n - 1));
        }
#pragma unroll
        for (int k = 0; k < kReadPerThread; ++k) {
            acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
        }
    }
    if (acc == 0x9e3779b9u) {
        *sink = acc;
    }
}
// The same read with ordinary (temporal) loads, for the comparison the weight streams
// are tuned on: the kernels mark their streamed weights non-temporal.
__global__ __launch_bounds__(kReadThreads) void stream_read_plain_kernel(const uint4 *__restrict__ src, size_t n,
                                                                         uint32_t *__restrict__ sink) {
    const size_t stride = size_t(gridDim.x) * kReadThreads * kReadPerThread;
    uint32_t acc = 0;
    for (size_t base = size_t(blockIdx.x) * kReadThreads * kReadPerThread + threadIdx.x; base < n; base += stride) {
        uint4 v[kReadPerThread];
#pragma unroll
        for (int k = 0; k < kReadPerThread; ++k) {
            const size_t i = base + size_t(k) * kReadThreads;
            v[k] = src[i < n ? i : n - 1];
        }
#pragma unroll
        for (int k = 0; k < kReadPerThread; ++k) {
            acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
        }
    }
    if (acc == 0x9e3779b9u) {
        *sink = acc;
    }
}

// ---- the cost of a kernel boundary: a chain of launches that each depend on the last ----
//
// Kernel i of a chain reads word[i % 2], which kernel i - 1 wrote, in every workgroup
// (the shape of a decode step, whose every kernel starts by reading what the previous
// one wrote), and workgroup 0 writes word[(i + 1) % 2] = that value + 1.  Nothing else
// is done, so the time per launch in a replayed graph is the boundary alone.
__global__ void boundary_kernel(uint32_t *word, uint32_t i, uint32_t *sink) {
    const uint32_t v = word[i % 2];
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        word[(i + 1) % 2] = v + 1;
    }
    if (v == 0xffffffffu) {  // never: keeps every workgroup's load live
        *sink = v;
    }
}

// ---- a device-wide handoff: a kernel boundary against a barrier inside one kernel ----
//
// 180 producer workgroups each write 16 floats (the shape of the 16-row matvec tiles);
// 32 consumers then each need all 2880 values (the shape of the router rows).  Across a
// kernel boundary the producers are one launch and the consumers the next.  Inside one
// launch each producer publishes its values with an agent-scope release fence and a flag
// (an epoch, so nothing is reset between launches); each consumer polls the 180 flags in
// parallel, boundedly, then takes an agent-scope acquire fence and reads.  Every
// workgroup of the one-launch form is resident at once (212 <= the CU count).
constexpr int kHandoffProducers = 180, kHandoffConsumers = 32, kHandoffThreads = 256, kHandoffValues = 2880;
constexpr unsigned kHandoffMaxSpin = 200000;

struct HandoffState {
    float data[kHandoffValues];
    unsigned flags[kHandoffProducers * 16];  // one flag per 64-byte line
    unsigned epoch, done, failures;
    float out[kHandoffConsumers];
};

__device__ inline void handoff_produce(HandoffState *st) {
    if (threadIdx.x < 16) {
        st->data[blockIdx.x * 16 + threadIdx.x] = float(blockIdx.x * 16 + threadIdx.x) * 0.5f;
    }
}

// Sums the values in a fixed order (exact: multiples of 0.5 below 2^22) and records it.
__device__ inline void handoff_consume(HandoffState *st, uint32_t consumer, bool ok) {
    __shared__ float red[kHandoffThreads];
    float s = 0.0f;
    for (int i = int(threadIdx.x); i < kHandoffValues; i += kHandoffThreads) {
        s += st->data[i];
    }
    red[threadIdx.x] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float a = 0.0f;
        for (int i = 0; i < kHandoffThreads; ++i) {
            a += red[i];
        }
        st->out[consumer] = ok ? a : -1.0f;
    }
}

__global__ __launch_bounds__(kHandoffThreads) void handoff_producers_kernel(HandoffState *st) {
    handoff_produce(st);
}

__global__ __launch_bounds__(kHandoffThreads) void handoff_consumers_kernel(HandoffState *st) {
    handoff_consume(st, blockIdx.x, true);
}

// Inside one launch without fences: each producer writes its values with agent-scope
// stores (written through past its XCD's L2), waits for them to complete, then writes
// its flag the same way; each consumer polls the flags and reads the values with
// agent-scope loads (past its own L2), so no L2 is written back or invalidated.
__global__ __launch_bounds__(kHandoffThreads) void handoff_in_kernel_nofence(HandoffState *st) {
    const unsigned epoch = __hip_atomic_load(&st->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
    if (blockIdx.x < uint32_t(kHandoffProducers)) {
        if (threadIdx.x < 64) {
            if (threadIdx.x < 16) {
                const uint32_t i = blockIdx.x * 16 + threadIdx.x;
                __hip_atomic_store(&st->data[i], float(i) * 0.5f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            if (threadIdx.x == 0) {
                __hip_atomic_store(&st->flags[blockIdx.x * 16], epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        return;
    }
    __shared__ int all;
    __shared__ float red[kHandoffThreads];
    if (threadIdx.x == 0) {
        all = 1;
    }
    __syncthreads();
    if (threadIdx.x < uint32_t(kHandoffProducers)) {
        unsigned spins = 0;
        while (__hip_atomic_load(&st->flags[threadIdx.x * 16], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != epoch &&
               spins < kHandoffMaxSpin) {
            __builtin_amdgcn_s_sleep(1);
            ++spins;
        }
        if (spins == kHandoffMaxSpin) {
            all = 0;
        }
    }
    __syncthreads();
    const uint32_t consumer = blockIdx.x - kHandoffProducers;
    // all of a thread's loads requested before the first is used: as a loop of loads
    // each added to the sum, every load waited for the one before (a round trip each)
    constexpr int kPer = (kHandoffValues + kHandoffThreads - 1) / kHandoffThreads;
    float v[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = min(int(threadIdx.x) + k * kHandoffThreads, kHandoffValues - 1);
        v[k] = __hip_atomic_load(&st->data[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        sum += int(threadIdx.x) + k * kHandoffThreads < kHandoffValues ? v[k] : 0.0f;
    }
    red[threadIdx.x] = sum;
    __syncthreads();
    if (threadIdx.x == 0) {
        float a = 0.0f;
        for (int i = 0; i < kHandoffThreads; ++i) {
            a += red[i];
        }
        st->out[consumer] = all ? a : -1.0f;
        if (!all) {
            __hip_atomic_fetch_add(&st->failures, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        const unsigned d = __hip_atomic_fetch_add(&st->done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (d == unsigned(kHandoffConsumers - 1)) {
            __hip_atomic_store(&st->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&st->epoch, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

__global__ __launch_bounds__(kHandoffThreads) void handoff_in_kernel(HandoffState *st) {
    const unsigned epoch = __hip_atomic_load(&st->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
    if (blockIdx.x < uint32_t(kHandoffProducers)) {
        handoff_produce(st);
        __syncthreads();
        if (threadIdx.x == 0) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            __hip_atomic_store(&st->flags[blockIdx.x * 16], epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    __shared__ int all;
    if (threadIdx.x == 0) {
        all = 1;
    }
    __syncthreads();
    if (threadIdx.x < uint32_t(kHandoffProducers)) {
        unsigned spins = 0;
        while (__hip_atomic_load(&st->flags[threadIdx.x * 16], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != epoch &&
               spins < kHandoffMaxSpin) {
            __builtin_amdgcn_s_sleep(1);
            ++spins;
        }
        if (spins == kHandoffMaxSpin) {
            all = 0;  // gave up: recorded as a failure, never waits longer
        }
    }
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    const uint32_t consumer = blockIdx.x - kHandoffProducers;
    handoff_consume(st, consumer, all != 0);
    if (threadIdx.x == 0) {
        if (!all) {
            __hip_atomic_fetch_add(&st->failures, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        const unsigned d = __hip_atomic_fetch_add(&st->done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (d == unsigned(kHandoffConsumers - 1)) {  // the last consumer opens the next epoch
            __hip_atomic_store(&st->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&st->epoch, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}
}  // namespace

namespace ttl {
int set_error(int code, const char *fmt, ...) {
    va_list args;
    va_start(args, fmt);
    std::vsnprintf(last_error, sizeof(last_error), fmt, args);
    va_end(args);
    return code;
}

int hip_fail(hipError_t err, const char *what) {
    return set_error(err == hipErrorOutOfMemory ? TTL_ERR_MEMORY : TTL_ERR_HIP, "%s: %s", what,
                     hipGetErrorString(err));
}
}  // namespace ttl

extern "C" {

const char *ttl_last_error(void) {
    return last_error;
}

int ttl_create(int device, ttl_ctx **out) {
    TTL_REQUIRE(out != nullptr, TTL_ERR_INVALID, "ttl_create: null output pointer");
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= device || device < 0) {
        return ttl::set_error(TTL_ERR_NO_DEVICE, "ttl_create: no HIP device %d (found %d)", device, count);
    }
    hipDeviceProp_t prop;
    TTL_HIP(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        return ttl::set_error(TTL_ERR_NO_DEVICE, "ttl_create: device %d is %s, this library is built for gfx950",
                              device, prop.gcnArchName);
    }
    TTL_HIP(hipSetDevice(device));
    ttl_ctx *ctx = new ttl_ctx;
    ctx->device = device;
    ctx->compute_units = prop.multiProcessorCount;
    ctx->hbm_bytes = double(prop.totalGlobalMem);
    std::snprintf(ctx->name, sizeof(ctx->name), "%s (%s)", prop.name, prop.gcnArchName);
    hipError_t err = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (err == hipSuccess) {
        err = hipEventCreate(&ctx->timer_start);
    }
    if (err == hipSuccess) {
        err = hipEventCreate(&ctx->timer_stop);
    }
    if (err == hipSuccess) {
        err = hipMalloc(&ctx->moe_workspace, ttl::moe_workspace_bytes());
    }
    if (err == hipSuccess) {
        err = hipMemset(ctx->moe_workspace, 0, ttl::moe_workspace_bytes());
    }
    if (err != hipSuccess) {
        ttl_destroy(ctx);
        return ttl::hip_fail(err, "ttl_create");
    }
    const int rc = ttl::attention_scratch_init(device);  // the device is current here
    if (rc != TTL_OK) {
        ttl_destroy(ctx);
        return rc;
    }
    *out = ctx;
    return TTL_OK;
}

void ttl_destroy(ttl_ctx *ctx) {
    if (!ctx) {
        return;
    }
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) {
        (void)hipStreamSynchronize(ctx->stream);
    }
    if (ctx->timer_start) {
        (void)hipEventDestroy(ctx->timer_start);
    }
    if (ctx->timer_stop) {
        (void)hipEventDestroy(ctx->timer_stop);
    }
    if (ctx->stream) {
        (void)hipStreamDestroy(ctx->stream);
    }
    if (ctx->moe_workspace) {
        (void)hipFree(ctx->moe_workspace);
    }
    delete ctx;
}

int ttl_sync(ttl_ctx *ctx) {
    TTL_REQUIRE(ctx, TTL_ERR_INVALID, "ttl_sync: null context");
    TTL_HIP(hipStreamSynchronize(ctx->stream));
    return TTL_OK;
}

int ttl_device_info(ttl_ctx *ctx, char *name, size_t name_bytes, int *compute_units, double *hbm_bytes) {
    TTL_REQUIRE(ctx, TTL_ERR_INVALID, "ttl_device_info: null context");
    if (name && name_bytes) {
        std::snprintf(name, name_bytes, "%s", ctx->name);
    }
    if (compute_units) {
        *compute_units = ctx->compute_units;
    }
    if (hbm_bytes) {
        *hbm_bytes = ctx->hbm_bytes;
    }
    return TTL_OK;
}

int ttl_malloc(ttl_ctx *ctx, size_t bytes, void **dev) {
    TTL_REQUIRE(ctx && dev, TTL_ERR_INVALID, "ttl_malloc: null argument");
    *dev = nullptr;
    TTL_HIP(hipSetDevice(ctx->device));
    TTL_HIP(hipMalloc(dev, bytes ? bytes : 1));
    return TTL_OK;
}

int ttl_free(ttl_ctx *ctx, void *dev) {
    TTL_REQUIRE(ctx, TTL_ERR_INVALID, "ttl_free: null context");
    if (dev) {
        TTL_HIP(hipStreamSynchronize(ctx->stream));
        TTL_HIP(hipFree(dev));
    }
    return TTL_OK;
}

int ttl_memcpy_h2d(ttl_ctx *ctx, void *dst_dev, const void *src, size_t bytes) {
    TTL_REQUIRE(ctx && (bytes == 0 || (dst_dev && src)), TTL_ERR_INVALID, "ttl_memcpy_h2d: null argument");
    TTL_HIP(hipMemcpyAsync(dst_dev, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    // The source is pageable host memory owned by the caller; wait so it may be reused.
    TTL_HIP(hipStreamSynchronize(ctx->stream));
    return TTL_OK;
}

int ttl_memcpy_d2h(ttl_ctx *ctx, void *dst, const void *src_dev, size_t bytes) {
    TTL_REQUIRE(ctx && (bytes == 0 || (dst && src_dev)), TTL_ERR_INVALID, "ttl_memcpy_d2h: null argument");
    TTL_HIP(hipMemcpyAsync(dst, src_dev, bytes, hipMemcpyDeviceToHost, ctx->stream));
    TTL_HIP(hipStreamSynchronize(ctx->stream));
    return TTL_OK;
}

int ttl_memcpy_d2d(ttl_ctx *ctx, void *dst_dev, const void *src_dev, size_t bytes) {
    TTL_REQUIRE(ctx && (bytes == 0 || (dst_dev && src_dev)), TTL_ERR_INVALID, "ttl_memcpy_d2d: null argument");
    const bool aligned = ((uintptr_t(dst_dev) | uintptr_t(src_dev) | bytes) & 15) == 0;
    if (!aligned) {
        TTL_HIP(hipMemcpyAsync(dst_dev, src_dev, bytes, hipMemcpyDeviceToDevice, ctx->stream));
        return TTL_OK;
    }
    if (bytes == 0) {
        return TTL_OK;
    }
    const size_t n = bytes / 16;
    const unsigned threads = 256;
    const unsigned blocks = unsigned(std::min<size_t>(ttl::blocks_for(n, threads), 8192));
    copy16_kernel<<<blocks, threads, 0, ctx->stream>>>((const uint4 *)src_dev, (uint4 *)dst_dev, n);
    TTL_LAUNCHED("copy16_kernel");
    return TTL_OK;
}

int ttl_fill_bytes(ttl_ctx *ctx, void *dst_dev, uint8_t value, size_t bytes) {
    TTL_REQUIRE(ctx && (bytes == 0 || dst_dev), TTL_ERR_INVALID, "ttl_fill_bytes: null argument");
    if (bytes == 0) {
        return TTL_OK;
    }
    const unsigned threads = 256;
    const unsigned blocks = unsigned(std::min<size_t>(ttl::blocks_for(bytes, threads), 4096));
    fill_bytes_kernel<<<blocks, threads, 0, ctx->stream>>>((uint8_t *)dst_dev, value, bytes);
    TTL_LAUNCHED("fill_bytes_kernel");
    return TTL_OK;
}

int ttl_stream_read(ttl_ctx *ctx, const void *src_dev, size_t bytes, uint32_t *sink_dev) {
    TTL_REQUIRE(ctx && src_dev && sink_dev, TTL_ERR_INVALID, "ttl_stream_read: null argument");
    TTL_REQUIRE(bytes >= 16 && bytes % 16 == 0, TTL_ERR_SHAPE, "ttl_stream_read: bytes must be a positive multiple of 16");
    TTL_REQUIRE((reinterpret_cast<uintptr_t>(src_dev) & 15) == 0, TTL_ERR_INVALID,
                "ttl_stream_read: source must be 16-byte aligned");
    const size_t words = bytes / 16;
    const size_t per_block = size_t(kReadThreads) * kReadPerThread;
    const size_t blocks = std::min((words + per_block - 1) / per_block, size_t(kReadBlocks));
    stream_read_kernel<<<unsigned(blocks), kReadThreads, 0, ctx->stream>>>(static_cast<const uint4 *>(src_dev), words,
                                                                       sink_dev);
    TTL_LAUNCHED("stream_read_kernel");
    return TTL_OK;
}

int ttl_stream_read_plain(ttl_ctx *ctx, const void *src_dev, size_t bytes, uint32_t *sink_dev) {
    TTL_REQUIRE(ctx && src_dev && sink_dev, TTL_ERR_INVALID, "ttl_stream_read_plain: null argument");
    TTL_REQUIRE(bytes >= 16 && bytes % 16 == 0, TTL_ERR_SHAPE,
                "ttl_stream_read_plain: bytes must be a positive multiple of 16");
    TTL_REQUIRE((reinterpret_cast<uintptr_t>(src_dev) & 15) == 0, TTL_ERR_INVALID,
                "ttl_stream_read_plain: source must be 16-byte aligned");
    const size_t words = bytes / 16;
    const size_t per_block = size_t(kReadThreads) * kReadPerThread;
    const size_t blocks = std::min((words + per_block - 1) / per_block, size_t(kReadBlocks));
    stream_read_plain_kernel<<<unsigned(blocks), kReadThreads, 0, ctx->stream>>>(static_cast<const uint4 *>(src_dev),
                                                                             words, sink_dev);
    TTL_LAUNCHED("stream_read_plain_kernel");
    return TTL_OK;
}

int ttl_measure_boundary(ttl_ctx *ctx, uint32_t launches, uint32_t blocks, uint32_t threads, float *us_per_kernel,
                         uint32_t *wrong) {
    TTL_REQUIRE(ctx && us_per_kernel && wrong, TTL_ERR_INVALID, "ttl_measure_boundary: null argument");
    TTL_REQUIRE(launches >= 2 && launches <= 1000, TTL_ERR_INVALID, "ttl_measure_boundary: 2..1000 launches");
    TTL_REQUIRE(blocks >= 1 && blocks <= 65536 && threads >= 64 && threads <= 1024 && threads % 64 == 0,
                TTL_ERR_INVALID, "ttl_measure_boundary: 1..65536 workgroups of 64..1024 threads (a multiple of 64)");
    uint32_t *words = nullptr;
    TTL_HIP(hipMalloc(&words, 4 * sizeof(uint32_t)));
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int rc = TTL_OK;
    const auto fail = [&](hipError_t err, const char *what) {
        if (rc == TTL_OK && err != hipSuccess) {
            rc = ttl::hip_fail(err, what);
        }
    };
    fail(hipMemsetAsync(words, 0, 4 * sizeof(uint32_t), ctx->stream), "hipMemsetAsync");
    fail(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (rc == TTL_OK) {
        fail(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        // an even chain, so every replay starts from word[0]
        const uint32_t n = launches + launches % 2;
        for (uint32_t i = 0; i < n && rc == TTL_OK; ++i) {
            boundary_kernel<<<blocks, threads, 0, ctx->stream>>>(words, i, words + 2);
        }
        fail(hipStreamEndCapture(ctx->stream, &graph), "hipStreamEndCapture");
        launches = n;
    }
    if (rc == TTL_OK) {
        fail(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    }
    constexpr int kReps = 20;
    float ms = 0.0f;
    if (rc == TTL_OK) {
        fail(hipGraphLaunch(exec, ctx->stream), "hipGraphLaunch");
        fail(hipEventRecord(ctx->timer_start, ctx->stream), "hipEventRecord");
        for (int r = 0; r < kReps && rc == TTL_OK; ++r) {
            fail(hipGraphLaunch(exec, ctx->stream), "hipGraphLaunch");
        }
        fail(hipEventRecord(ctx->timer_stop, ctx->stream), "hipEventRecord");
        fail(hipEventSynchronize(ctx->timer_stop), "hipEventSynchronize");
        fail(hipEventElapsedTime(&ms, ctx->timer_start, ctx->timer_stop), "hipEventElapsedTime");
    }
    uint32_t host[4] = {0, 0, 0, 0};
    if (rc == TTL_OK) {
        fail(hipMemcpy(host, words, sizeof host, hipMemcpyDeviceToHost), "hipMemcpy");
    }
    if (exec) {
        (void)hipGraphExecDestroy(exec);
    }
    if (graph) {
        (void)hipGraphDestroy(graph);
    }
    (void)hipFree(words);
    if (rc != TTL_OK) {
        return rc;
    }
    // every kernel of every replay added one along the chain
    *wrong = host[0] == launches * uint32_t(kReps + 1) ? 0u : 1u;
    *us_per_kernel = ms * 1000.0f / float(kReps * launches);
    return TTL_OK;
}

int ttl_measure_handoff(ttl_ctx *ctx, int mode, uint32_t launches, float *us_per_handoff, uint32_t *wrong) {
    TTL_REQUIRE(ctx && us_per_handoff && wrong, TTL_ERR_INVALID, "ttl_measure_handoff: null argument");
    TTL_REQUIRE(mode >= 0 && mode <= 2, TTL_ERR_INVALID, "ttl_measure_handoff: mode must be 0, 1 or 2");
    TTL_REQUIRE(launches >= 1 && launches <= 1000, TTL_ERR_INVALID, "ttl_measure_handoff: 1..1000 launches");
    TTL_REQUIRE(ctx->compute_units >= kHandoffProducers + kHandoffConsumers, TTL_ERR_SHAPE,
                "ttl_measure_handoff: needs %d resident workgroups", kHandoffProducers + kHandoffConsumers);
    HandoffState *st = nullptr;
    TTL_HIP(hipMalloc(&st, sizeof(HandoffState)));
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int rc = TTL_OK;
    const auto fail = [&](hipError_t err, const char *what) {
        if (rc == TTL_OK && err != hipSuccess) {
            rc = ttl::hip_fail(err, what);
        }
    };
    fail(hipMemsetAsync(st, 0, sizeof(HandoffState), ctx->stream), "hipMemsetAsync");
    fail(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    // one graph of `launches` handoffs, replayed: first untimed, then timed
    if (rc == TTL_OK) {
        fail(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        for (uint32_t i = 0; i < launches && rc == TTL_OK; ++i) {
            if (mode == 0) {
                handoff_producers_kernel<<<kHandoffProducers, kHandoffThreads, 0, ctx->stream>>>(st);
                handoff_consumers_kernel<<<kHandoffConsumers, kHandoffThreads, 0, ctx->stream>>>(st);
            } else if (mode == 1) {
                handoff_in_kernel<<<kHandoffProducers + kHandoffConsumers, kHandoffThreads, 0, ctx->stream>>>(st);
            } else {
                handoff_in_kernel_nofence<<<kHandoffProducers + kHandoffConsumers, kHandoffThreads, 0,
                                            ctx->stream>>>(st);
            }
        }
        fail(hipStreamEndCapture(ctx->stream, &graph), "hipStreamEndCapture");
    }
    if (rc == TTL_OK) {
        fail(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    }
    constexpr int kReps = 20;
    float ms = 0.0f;
    if (rc == TTL_OK) {
        fail(hipGraphLaunch(exec, ctx->stream), "hipGraphLaunch");
        fail(hipEventRecord(ctx->timer_start, ctx->stream), "hipEventRecord");
        for (int r = 0; r < kReps && rc == TTL_OK; ++r) {
            fail(hipGraphLaunch(exec, ctx->stream), "hipGraphLaunch");
        }
        fail(hipEventRecord(ctx->timer_stop, ctx->stream), "hipEventRecord");
        fail(hipEventSynchronize(ctx->timer_stop), "hipEventSynchronize");
        fail(hipEventElapsedTime(&ms, ctx->timer_start, ctx->timer_stop), "hipEventElapsedTime");
    }
    HandoffState host;
    if (rc == TTL_OK) {
        fail(hipMemcpy(&host, st, sizeof host, hipMemcpyDeviceToHost), "hipMemcpy");
    }
    if (exec) {
        (void)hipGraphExecDestroy(exec);
    }
    if (graph) {
        (void)hipGraphDestroy(graph);
    }
    (void)hipFree(st);
    if (rc != TTL_OK) {
        return rc;
    }
    const float expected = 0.5f * float(kHandoffValues) * float(kHandoffValues - 1) / 2.0f;
    uint32_t bad = host.failures;
    for (int c = 0; c < kHandoffConsumers; ++c) {
        bad += host.out[c] != expected ? 1u : 0u;
    }
    *wrong = bad;
    *us_per_handoff = ms * 1000.0f / float(kReps * launches);
    return TTL_OK;
}

int ttl_capture_begin(ttl_ctx *ctx) {
    TTL_REQUIRE(ctx, TTL_ERR_INVALID, "ttl_capture_begin: null context");
    TTL_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    return TTL_OK;
}

int ttl_capture_end(ttl_ctx *ctx, ttl_graph **out) {
    TTL_REQUIRE(ctx && out, TTL_ERR_INVALID, "ttl_capture_end: null argument");
    *out = nullptr;
    hipGraph_t graph = nullptr;
    TTL_HIP(hipStreamEndCapture(ctx->stream, &graph));
    hipGraphExec_t exec = nullptr;
    const hipError_t err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (err != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return ttl::hip_fail(err, "hipGraphInstantiate");
    }
    *out = new ttl_graph{graph, exec};
    return TTL_OK;
}

int ttl_graph_launch(ttl_ctx *ctx, ttl_graph *graph) {
    TTL_REQUIRE(ctx && graph, TTL_ERR_INVALID, "ttl_graph_launch: null argument");
    TTL_HIP(hipGraphLaunch(graph->exec, ctx->stream));
    return TTL_OK;
}

void ttl_graph_free(ttl_graph *graph) {
    if (graph) {
        (void)hipGraphExecDestroy(graph->exec);
        (void)hipGraphDestroy(graph->graph);
        delete graph;
    }
}

int ttl_timer_start(ttl_ctx *ctx) {
    TTL_REQUIRE(ctx, TTL_ERR_INVALID, "ttl_timer_start: null context");
    TTL_HIP(hipEventRecord(ctx->timer_start, ctx->stream));
    return TTL_OK;
}

int ttl_timer_stop(ttl_ctx *ctx, float *ms) {
    TTL_REQUIRE(ctx && ms, TTL_ERR_INVALID, "ttl_timer_stop: null argument");
    TTL_HIP(hipEventRecord(ctx->timer_stop, ctx->stream));
    TTL_HIP(hipEventSynchronize(ctx->timer_stop));
    TTL_HIP(hipEventElapsedTime(ms, ctx->timer_start, ctx->timer_stop));
    return TTL_OK;
}

}  // extern "C"
