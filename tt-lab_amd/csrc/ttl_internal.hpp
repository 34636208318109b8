// Internal definitions shared by the HIP sources of the gfx950 backend.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "../../include/ttlab_hip.h"

struct ttl_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t timer_start = nullptr;
    hipEvent_t timer_stop = nullptr;
    void *moe_workspace = nullptr;  // device ttl::MoeWorkspace, zeroed at creation
    int compute_units = 0;
    double hbm_bytes = 0.0;
    char name[128] = {};
};

struct ttl_graph {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

// MXFP4 tensor in the repacked layout (see mx:: constants).
struct ttl_mxfp4 {
    uint32_t rows = 0;
    uint32_t cols = 0;
    uint32_t experts = 0;
    uint32_t tiles = 0;          // rows / mx::tile_rows per expert
    uint8_t *codes = nullptr;    // [experts][tiles][blocks][tile_rows][16 B]
    uint8_t *scales = nullptr;   // [experts][tiles][lanes_k][tile_rows][scale_pad]
    size_t code_bytes = 0;
    size_t scale_bytes = 0;
    // Per expert: some block has E8M0 scale 255, or scale 0 with a nonzero code.  The
    // bf16 conversion of the MFMA kernels has no exact value for those (2^-127 is an
    // f32 subnormal scale, 2^128 none at all), so the batched entry points refuse such
    // experts; the matvec kernels decode every scale exactly.
    std::vector<uint8_t> edge_experts;
    bool edge_scales() const {
        for (uint8_t f : edge_experts) {
            if (f) {
                return true;
            }
        }
        return false;
    }
    // Per expert: some block with a nonzero code has an E8M0 scale outside 114..140, where
    // E2M1 times the scale is not always a normal f16 (the f16 decode of the prefill's down
    // GEMM is exact only inside; such tensors take the bf16 decode).
    std::vector<uint8_t> f16_inexact_experts;
    bool f16_exact() const {
        if (f16_inexact_experts.size() != experts) {
            return false;  // not computed for this tensor
        }
        for (uint8_t f : f16_inexact_experts) {
            if (f) {
                return false;
            }
        }
        return true;
    }
};

// Q8_0 tensor in the repacked layout (see q8:: constants in ttl_q8_tile.hpp): rows of
// GGUF Q8_0 blocks (fp16 scale + 32 int8), optionally permuted at upload.
struct ttl_q8 {
    uint32_t rows = 0;
    uint32_t cols = 0;
    uint32_t tiles = 0;          // rows / 16
    uint8_t *codes = nullptr;    // [tiles][blocks][2 halves][16 rows][16 B]
    uint16_t *scales = nullptr;  // [tiles][4 lanes_k][16 rows][scale_pad] fp16
    uint16_t *row_scales = nullptr;  // [rows][blocks] fp16, for the batched matmul
    size_t code_bytes = 0;
    size_t scale_bytes = 0;
};

namespace ttl {

size_t moe_workspace_bytes();
// Looks up the device address of the attention partials' static array (ttl_attn.hip)
// for `device`, which must be current; once per device.
int attention_scratch_init(int device);
// Batched router of moe_batch (ttl_moe.hip): per-token exact rows in `scratch`
// (router_scratch_bytes() each), indices/weights [count][used].
size_t router_scratch_bytes();
int launch_router_batch(ttl_ctx *ctx, const ttl_moe_layer &L, const float *x, uint32_t count, void *scratch,
                        int32_t *indices, float *weights);

// The shift k of each of `rows` f32 rows (`cols` values each, a multiple of 4 and at most
// 4096, rows `stride` floats apart, 16-byte aligned) for their two f16 planes: k of the
// row's largest finite magnitude (mf::row_shift), into shift[rows] (ttl_prefill.hip).
int launch_row_shifts(hipStream_t stream, const float *x, uint32_t stride, uint32_t rows, uint32_t cols,
                       int32_t *shift);

int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t err, const char *what);

// Launch configuration helper: blocks needed for n items.
inline unsigned blocks_for(size_t n, unsigned threads) {
    return unsigned((n + threads - 1) / threads);
}

// A 16-byte load marked non-temporal (the instruction's nt bit), for weights that are
// streamed once per pass: a plain read of 1.16 GB ran at 7.0 TB/s this way against
// 6.2 TB/s with ordinary loads (gfx950, 1024-4096 workgroups, 4 or 8 loads in flight).
// Only for loads whose wave covers whole 128-byte lines: Q8_0 tiles read as the two
// 16-byte halves of each 32-byte lane record got slower with it (QKV 8.7 -> 9.4 us),
// hence their layout of halves (q8::code_offset).  Not for data re-read soon: the
// sliding-window attention's cached K/V rows (re-read every token) went from 5.7 to
// 7.7 us per launch with it.
__device__ __forceinline__ uint4 load_stream(const uint4 *p) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(w[0], w[1], w[2], w[3]);
}

}  // namespace ttl

#define TTL_HIP(call)                                  \
    do {                                               \
        hipError_t ttl_err_ = (call);                  \
        if (ttl_err_ != hipSuccess) {                  \
            return ttl::hip_fail(ttl_err_, #call);     \
        }                                              \
    } while (0)

#define TTL_LAUNCHED(what)                             \
    do {                                               \
        hipError_t ttl_err_ = hipGetLastError();       \
        if (ttl_err_ != hipSuccess) {                  \
            return ttl::hip_fail(ttl_err_, what);      \
        }                                              \
    } while (0)

#define TTL_REQUIRE(cond, code, ...)                   \
    do {                                               \
        if (!(cond)) {                                 \
            return ttl::set_error(code, __VA_ARGS__);  \
        }                                              \
    } while (0)

// Repacked MXFP4 layout.  A tile is 16 consecutive rows of one expert; within a
// tile the 16-byte code chunks are ordered [block][row], so the 64 lanes of a
// wave that read blocks 4i..4i+3 of the tile's 16 rows touch 1 KiB of contiguous
// memory.  Scale bytes are ordered so that each lane's 23 scales (blocks
// kl, kl+4, ..., kl+88 of its row) are 24 contiguous bytes.
namespace mx {
constexpr int tile_rows = 16;
constexpr int cols = 2880;
constexpr int blocks = cols / 32;                             // 90 blocks per row
constexpr int lanes_k = 4;                                    // lanes sharing a row
constexpr int iters = (blocks + lanes_k - 1) / lanes_k;       // 23
constexpr int scale_pad = 24;                                 // per-lane scale bytes
constexpr size_t tile_code_bytes = size_t(blocks) * tile_rows * 16;          // 23040
constexpr size_t tile_scale_bytes = size_t(lanes_k) * tile_rows * scale_pad; // 1536
constexpr uint8_t pad_scale = 127;                            // scale of padding blocks
// One 32-bit word per expert after the scale plane, set by the repack: bit 0 for the edge
// scales (ttl_mxfp4::edge_experts), bit 1 for scales outside the f16 decode's range
// (ttl_mxfp4::f16_inexact_experts).
inline size_t edge_flag_bytes(uint32_t experts) {
    return (size_t(experts) * 4 + 15) / 16 * 16;
}
// Zero bytes after the last tile: iterations past the row end (blocks 90..95) read
// there unconditionally (their x is zero, and E2M1 codes are all finite).
constexpr size_t tail_pad_bytes = size_t(24 * lanes_k - blocks) * tile_rows * 16;  // 1536: up to block 95

__host__ __device__ inline size_t code_chunk(size_t tile_index, uint32_t block, uint32_t row) {
    return (tile_index * blocks + block) * tile_rows + row;
}
__host__ __device__ inline size_t scale_offset(size_t tile_index, uint32_t block, uint32_t row) {
    return tile_index * tile_scale_bytes + (size_t(block % lanes_k) * tile_rows + row) * scale_pad + block / lanes_k;
}
}  // namespace mx

// Synthetic-input generator shared with oracle/ttlab_oracle.c (same arithmetic).
namespace synth {
__host__ __device__ inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__host__ __device__ inline uint64_t hash(uint64_t seed, uint64_t stream, uint64_t index) {
    return mix64(seed + stream * 0xD1342543DE82EF95ull + (index + 1) * 0x9E3779B97F4A7C15ull);
}
}  // namespace synth
