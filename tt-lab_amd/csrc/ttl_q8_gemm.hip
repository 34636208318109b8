// Batched Q8_0 matmul on MFMA: matmul_add_q8_0 (tensor.cpp:529-566) for a batch of
// tokens, as GptOssModel::prefill runs the attention projections (model.cpp:493-498,
// 519-520).
//
// Operands of v_mfma_f32_16x16x32_f16 (D = A B + C; lane l holds 8 f16 of A row
// l%16 and of B column l%16 for the K offsets of lane group g = l/16, and receives D
// rows 4g..4g+3 of column l%16):
//  - one K step is one Q8_0 block of 32 columns; lane group g holds offsets 8g..8g+7;
//  - A is 16 tokens: token t's f32 activations times 2^k_t as two f16 planes
//    (mf::split_f16x2, k_t = mf::row_shift of the row's largest finite |x|), staged
//    through LDS;
//  - B is 16 weight rows: the int8 codes, exact in f16 (|q| <= 128 < 2^11);
//  - D[token][row]: a lane holds four tokens of one row, so the block's fp16 scale is
//    one value per lane, applied after the block: acc += d * (A0 B + A1 B).
// Every product q x is exact; the MFMA sums a block's products in f32 and d times that
// sum is added to the accumulator, all times 2^k_t, which the store takes back (powers
// of two: the same roundings as unscaled).  The two planes hold each activation to
// 2^-22 of itself (to 2^-39 of the row's largest below 2^-17 of it).  The reference sums
// the products sequentially from the bias (d q rounds to nothing: it has at most 19
// significant bits), so results agree to f32 rounding, not bit for bit.
//
// Workspace: token fragments [token tile of 64][plane][step][16-token sub-tile][lane][16 B]
// (steps past the last block -- K = 2880 has 90 blocks, padded to 92 -- hold zero tokens,
// and their row scales are zero), then the tokens' shifts k_t [tiles x 64] (int32), unless
// the caller passes them (ttl_matmul_q8_0_shifted).
#include "ttl_mfma.hpp"

#include <hip/hip_fp16.h>

namespace {

using mf::f16x8;
using mf::f32x4;

constexpr int kPlanes = 2;
constexpr int kSub = 4;  // 16-token sub-tiles per 64-token tile
constexpr int kTileTokens = 16 * kSub;
constexpr int kStageSteps = 2;  // K steps per LDS stage
constexpr int kWaves = 4;
// 16-row weight tiles per wave: one.  The projections have 2880 and 5120 rows, so more
// tiles per workgroup leave CUs idle at a 512-token prompt (measured: one tile per wave
// beat two and three in the layer-major prefill).
constexpr int kRowTiles = 1;
constexpr int kLook = 4;  // token fragments read from LDS this many ahead

template <int K>
struct Shape {
    static constexpr int blocks = K / 32;
    static constexpr int quads = (blocks + 3) / 4;
    static constexpr int steps = quads * 4;
    static constexpr int stages = steps / kStageSteps;
    static constexpr size_t plane_bytes = size_t(steps) * kSub * mf::frag_bytes;
    static constexpr size_t tile_bytes = kPlanes * plane_bytes;
    static constexpr int stage_frags = kPlanes * kStageSteps * kSub;
    static constexpr int stage_chunks = stage_frags * 64;  // 16-byte pieces
};

// Token fragments of one (step, tile): thread (sub-tile m, lane (t, g)) converts
// x[64 tile + 16 m + t][32 step + 8 g .. + 7] times 2^shift[token] (zero past the tokens
// or the row end).
template <int K>
__global__ __launch_bounds__(kSub * 64) void q8_gather_kernel(const float *__restrict__ x, uint32_t tokens,
                                                              const int32_t *__restrict__ shift,
                                                              uint8_t *__restrict__ frags) {
    using S = Shape<K>;
    const uint32_t step = blockIdx.x, tile = blockIdx.y;
    const uint32_t m = threadIdx.x / 64, lane = threadIdx.x % 64, g = lane / 16;
    const uint32_t token = tile * kTileTokens + m * 16 + lane % 16;
    const int k = shift[token < tokens ? token : 0];
    float v[8];
    if (token < tokens && step < uint32_t(S::blocks)) {
        const float4 *p = reinterpret_cast<const float4 *>(x + size_t(token) * K + step * 32 + 8 * g);
        const float4 lo = p[0], hi = p[1];
        v[0] = lo.x;
        v[1] = lo.y;
        v[2] = lo.z;
        v[3] = lo.w;
        v[4] = hi.x;
        v[5] = hi.y;
        v[6] = hi.z;
        v[7] = hi.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v[j] = 0.0f;
        }
    }
    uint4 out[kPlanes];
    mf::split_f16x2(v, k, out);
    uint8_t *dst = frags + size_t(tile) * S::tile_bytes + (size_t(step) * kSub + m) * mf::frag_bytes + lane * 16;
#pragma unroll
    for (int p = 0; p < kPlanes; ++p) {
        *reinterpret_cast<uint4 *>(dst + size_t(p) * S::plane_bytes) = out[p];
    }
}

// 8 int8 codes (K order) as f16, exact: code q's byte with its top bit flipped is
// u = q + 128, and the f16 with bits 0x6400 | u is 1024 + u, so (1024 + u) - 1152 = q
// (an exact f16 subtraction).  Dword k holds codes 2k (low half) and 2k + 1.
__device__ inline f16x8 int8_f16(uint2 c) {
    typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
    const f16x2v bias = {_Float16(1152.0f), _Float16(1152.0f)};
    f16x8 r;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t w = (k < 2 ? c.x : c.y) ^ 0x80808080u;
        const uint32_t b = k % 2 == 0 ? w : w >> 16;  // the two codes in bytes 0 and 1
        const uint32_t h = (b & 0xffu) | ((b & 0xff00u) << 8) | 0x64006400u;
        const f16x2v v = __builtin_bit_cast(f16x2v, h) - bias;
        r[2 * k] = v[0];
        r[2 * k + 1] = v[1];
    }
    return r;
}

struct GemmArgs {
    const uint8_t *codes;        // repacked [tiles][blocks][2 halves][16 rows][16 B]
    const uint16_t *row_scales;  // [rows][steps] fp16 (zero past the blocks, q8::row_scale_stride)
    const float *bias;           // [rows] or null
    const float *residual;       // [tokens][rows] or null
    float *out;                  // [tokens][rows]
    const uint8_t *frags;        // token fragments
    const int32_t *shift;        // [tokens] the tokens' k (fragments hold x 2^k)
    uint32_t rows, row_tiles, tokens;
};

// One workgroup: a 64-token tile x 4 * kRowTiles weight-row tiles; wave w takes row
// tiles (group * 4 + w) * kRowTiles + j.  Token fragments go through LDS in stages of two K
// steps (double-buffered); each wave's weight codes and scales are requested one
// quad (4 steps) ahead.
template <int K>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2))) void q8_gemm_kernel(GemmArgs a) {
    using S = Shape<K>;
    constexpr int kThreads = kWaves * 64;
    constexpr int kPer = S::stage_chunks / kThreads;
    static_assert(S::stage_chunks % kThreads == 0, "the stager moves whole pieces");
    __shared__ mf::u32x4 lds[2][S::stage_chunks];
    const uint32_t t = threadIdx.x, wave = t / 64, lane = t % 64, n = lane % 16, g = lane / 16;
    const uint32_t tile = blockIdx.y;
    const uint8_t *frags = a.frags + size_t(tile) * S::tile_bytes;

    // this wave's weight row tiles (tiles past the matrix re-read tile 0; not written)
    const uint8_t *cp[kRowTiles];
    const uint16_t *sp[kRowTiles];
    bool ok[kRowTiles];
    uint32_t row[kRowTiles];
#pragma unroll
    for (int j = 0; j < kRowTiles; ++j) {
        const uint32_t rt = (blockIdx.x * kWaves + wave) * kRowTiles + j;
        ok[j] = rt < a.row_tiles;
        const uint32_t rts = ok[j] ? rt : 0;
        row[j] = rts * 16 + n;
        // bytes 8g..8g+7 of row n's block: half g / 2 (q8::code_offset), 8 (g % 2) into it
        cp[j] = a.codes + size_t(rts) * S::blocks * 512 + (g / 2) * 256 + n * 16 + 8 * (g % 2);
        sp[j] = a.row_scales + size_t(row[j]) * S::steps;
    }

    // stage j: K steps 2j, 2j+1 of all planes and sub-tiles, LDS order [plane][step][sub][lane]
    mf::u32x4 st[kPer];
    auto stage_load = [&](int j) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const uint32_t c = t + uint32_t(k) * kThreads;
            const uint32_t p = c / (kStageSteps * kSub * 64), within = c % (kStageSteps * kSub * 64);
            st[k] = *reinterpret_cast<const mf::u32x4 *>(frags + size_t(p) * S::plane_bytes +
                                                       size_t(j) * kStageSteps * kSub * mf::frag_bytes +
                                                       size_t(within) * 16);
        }
    };
    auto stage_store = [&](mf::u32x4 *dst) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            dst[t + uint32_t(k) * kThreads] = st[k];
        }
    };

    // weight codes and scales of one quad: [row tile][step], [row tile] (4 fp16)
    uint2 qc[2][kRowTiles][4];
    uint2 qs[2][kRowTiles];
    auto load_quad = [&](int q, uint2(&c)[kRowTiles][4], uint2(&s)[kRowTiles]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < kRowTiles; ++j) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t b = min(uint32_t(4 * q + k), uint32_t(S::blocks - 1));
                c[j][k] = *reinterpret_cast<const uint2 *>(cp[j] + size_t(b) * 512);
            }
            s[j] = *reinterpret_cast<const uint2 *>(sp[j] + 4 * q);
        }
    };

    // acc: the scaled sum so far.  The MFMAs of a K step go to cur; the scale FMAs of
    // a step run one step later, from pend (the previous step's sums) and pend_d, so the
    // VALU never waits on an MFMA result that was just issued.
    f32x4 acc[kSub][kRowTiles], cur[kSub][kRowTiles], pend[kSub][kRowTiles];
    float dcur[kRowTiles], pend_d[kRowTiles];
#pragma unroll
    for (int j = 0; j < kRowTiles; ++j) {
        dcur[j] = 0.0f;
        pend_d[j] = 0.0f;
#pragma unroll
        for (int m = 0; m < kSub; ++m) {
            acc[m][j] = f32x4{0.f, 0.f, 0.f, 0.f};
            pend[m][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }

    stage_load(0);
    load_quad(0, qc[0], qs[0]);
    stage_store(lds[0]);
    __syncthreads();
    stage_load(1);

    // the MFMAs of quad q (stages 2q, 2q+1) with its codes c and scales s
    auto compute_quad = [&](int q, const uint2(&c)[kRowTiles][4], const uint2(&s)[kRowTiles])
                            __attribute__((always_inline)) {
#pragma unroll
        for (int h = 0; h < 4 / kStageSteps; ++h) {
            const int stage = 2 * q + h;
            const mf::u32x4 *buf = lds[stage % 2];
            constexpr int SF = S::stage_frags;
            // fragment order within a stage: step, plane, sub-tile (the four sub-tiles'
            // MFMAs are independent, so consecutive MFMAs never wait on each other)
            auto frag = [&](int f) __attribute__((always_inline)) {
                const int ls = f / (kSub * kPlanes), p = (f / kSub) % kPlanes, m = f % kSub;
                return __builtin_bit_cast(f16x8, buf[((p * kStageSteps + ls) * kSub + m) * 64 + lane]);
            };
            f16x8 ring[kLook];
#pragma unroll
            for (int d = 0; d < kLook; ++d) {
                ring[d] = frag(d);
            }
            f16x8 w[kRowTiles];
#pragma unroll
            for (int f = 0; f < SF; ++f) {
                const f16x8 av = ring[f % kLook];
                if (f + kLook < SF) {
                    ring[f % kLook] = frag(f + kLook);
                }
                const int ls = f / (kSub * kPlanes), p = (f / kSub) % kPlanes, m = f % kSub;
                const int k = h * kStageSteps + ls;  // step within the quad
                if (f % (kSub * kPlanes) == 0) {
#pragma unroll
                    for (int j = 0; j < kRowTiles; ++j) {
                        w[j] = int8_f16(c[j][k]);
                        const uint32_t word = k < 2 ? s[j].x : s[j].y;
                        pend_d[j] = dcur[j];
                        dcur[j] = __half2float(__ushort_as_half(uint16_t(word >> (16 * (k % 2)))));
                    }
                }
#pragma unroll
                for (int j = 0; j < kRowTiles; ++j) {
                    cur[m][j] = mf::mfma(av, w[j], p == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : cur[m][j]);
                    if (p == kPlanes - 1) {
                        // the previous step's block sum, scaled by its fp16 d
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            acc[m][j][e] = fmaf(pend_d[j], pend[m][j][e], acc[m][j][e]);
                        }
                        // an empty statement that takes the sum in registers here: the
                        // compiler otherwise sinks these updates below the stage's MFMAs
                        // and keeps every block product live
                        asm volatile("" : "+v"(acc[m][j]));
                        pend[m][j] = cur[m][j];
                    }
                }
                // keep the ring's order: without this the scheduler hoists every LDS
                // read of the stage and runs out of registers
                __builtin_amdgcn_sched_barrier(0);
            }
            // end of stage: publish the next, fetch the one after
            if (stage + 1 < S::stages) {
                stage_store(lds[(stage + 1) % 2]);
            }
            __syncthreads();
            if (stage + 2 < S::stages) {
                stage_load(stage + 2);
            }
        }
    };

#pragma unroll 1
    for (int q = 0; q < S::quads; q += 2) {
        load_quad(min(q + 1, S::quads - 1), qc[1], qs[1]);
        compute_quad(q, qc[0], qs[0]);
        if (q + 1 < S::quads) {
            load_quad(min(q + 2, S::quads - 1), qc[0], qs[0]);
            compute_quad(q + 1, qc[1], qs[1]);
        }
    }
    // the last step's sums
#pragma unroll
    for (int j = 0; j < kRowTiles; ++j) {
#pragma unroll
        for (int m = 0; m < kSub; ++m) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc[m][j][e] = fmaf(dcur[j], pend[m][j][e], acc[m][j][e]);
            }
        }
    }

    // D rows 4g..4g+3 of sub-tile m are tokens; the lane's column is row[j]
    int ks[kSub][4];  // the shifts of the lane's 16 tokens (tokens past the count read token 0's)
#pragma unroll
    for (int m = 0; m < kSub; ++m) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t token = tile * kTileTokens + m * 16 + 4 * g + e;
            ks[m][e] = a.shift[token < a.tokens ? token : 0u];
        }
    }
#pragma unroll
    for (int j = 0; j < kRowTiles; ++j) {
        if (!ok[j]) {
            continue;
        }
        const float bv = a.bias ? a.bias[row[j]] : 0.0f;
#pragma unroll
        for (int m = 0; m < kSub; ++m) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t token = tile * kTileTokens + m * 16 + 4 * g + e;
                if (token < a.tokens) {
                    const size_t o = size_t(token) * a.rows + row[j];
                    const float sum = __builtin_amdgcn_ldexpf(acc[m][j][e], -ks[m][e]);
                    float v = a.bias ? bv + sum : sum;
                    if (a.residual) {
                        v = a.residual[o] + v;
                    }
                    a.out[o] = v;
                }
            }
        }
    }
}

template <int K>
size_t frag_bytes_for(uint32_t tokens) {
    return (size_t((tokens + kTileTokens - 1) / kTileTokens) * Shape<K>::tile_bytes + 255) & ~size_t(255);
}

template <int K>
size_t workspace_for(uint32_t tokens) {
    return frag_bytes_for<K>(tokens) + size_t((tokens + kTileTokens - 1) / kTileTokens) * kTileTokens * 4;
}

int matmul_q8_0(ttl_ctx *ctx, const ttl_q8 *w, const float *bias_dev, const float *x_dev, const int32_t *shift_dev,
                uint32_t tokens, const float *residual_dev, float *out_dev, void *workspace_dev,
                size_t workspace_bytes, const char *who) {
    TTL_REQUIRE(ctx && w && w->codes && w->row_scales && x_dev && out_dev && workspace_dev, TTL_ERR_INVALID,
                "%s: null argument", who);
    TTL_REQUIRE(w->cols == 2880 || w->cols == 4096, TTL_ERR_SHAPE, "%s: cols must be 2880 or 4096", who);
    TTL_REQUIRE(tokens < (1u << 20), TTL_ERR_SHAPE, "%s: at most %u tokens per call", who, (1u << 20) - 1);
    const size_t need = ttl_matmul_q8_0_workspace_bytes(tokens, w->cols);
    TTL_REQUIRE(workspace_bytes >= need, TTL_ERR_SHAPE, "%s: workspace of %zu bytes, %zu needed", who,
                workspace_bytes, need);
    TTL_REQUIRE((reinterpret_cast<uintptr_t>(x_dev) & 15) == 0 && (reinterpret_cast<uintptr_t>(workspace_dev) & 15) == 0,
                TTL_ERR_INVALID, "%s: x and the workspace must be 16-byte aligned", who);
    if (tokens == 0) {
        return TTL_OK;
    }
    const uint32_t tiles = (tokens + kTileTokens - 1) / kTileTokens;
    GemmArgs a;
    a.codes = w->codes;
    a.row_scales = w->row_scales;
    a.bias = bias_dev;
    a.residual = residual_dev;
    a.out = out_dev;
    a.frags = static_cast<const uint8_t *>(workspace_dev);
    int32_t *shift = reinterpret_cast<int32_t *>(static_cast<uint8_t *>(workspace_dev) +
                                                 (w->cols == 2880 ? frag_bytes_for<2880>(tokens)
                                                                  : frag_bytes_for<4096>(tokens)));
    if (shift_dev) {
        a.shift = shift_dev;
    } else {
        const int rc = ttl::launch_row_shifts(ctx->stream, x_dev, w->cols, tokens, w->cols, shift);
        if (rc != TTL_OK) {
            return rc;
        }
        a.shift = shift;
    }
    a.rows = w->rows;
    a.row_tiles = w->tiles;
    a.tokens = tokens;
    const uint32_t group = uint32_t(kWaves * kRowTiles);
    const dim3 grid((w->tiles + group - 1) / group, tiles);
    uint8_t *frags = static_cast<uint8_t *>(workspace_dev);
    if (w->cols == 2880) {
        q8_gather_kernel<2880><<<dim3(Shape<2880>::steps, tiles), kSub * 64, 0, ctx->stream>>>(x_dev, tokens, a.shift,
                                                                                               frags);
        q8_gemm_kernel<2880><<<grid, kWaves * 64, 0, ctx->stream>>>(a);
    } else {
        q8_gather_kernel<4096><<<dim3(Shape<4096>::steps, tiles), kSub * 64, 0, ctx->stream>>>(x_dev, tokens, a.shift,
                                                                                               frags);
        q8_gemm_kernel<4096><<<grid, kWaves * 64, 0, ctx->stream>>>(a);
    }
    TTL_LAUNCHED("q8 gemm kernels");
    return TTL_OK;
}

}  // namespace

extern "C" {

size_t ttl_matmul_q8_0_workspace_bytes(uint32_t tokens, uint32_t cols) {
    return cols == 4096 ? workspace_for<4096>(tokens) : workspace_for<2880>(tokens);
}

int ttl_matmul_q8_0(ttl_ctx *ctx, const ttl_q8 *w, const float *bias_dev, const float *x_dev, uint32_t tokens,
                    const float *residual_dev, float *out_dev, void *workspace_dev, size_t workspace_bytes) {
    return matmul_q8_0(ctx, w, bias_dev, x_dev, nullptr, tokens, residual_dev, out_dev, workspace_dev,
                       workspace_bytes, "ttl_matmul_q8_0");
}

int ttl_matmul_q8_0_shifted(ttl_ctx *ctx, const ttl_q8 *w, const float *bias_dev, const float *x_dev,
                            const int32_t *shift_dev, uint32_t tokens, const float *residual_dev, float *out_dev,
                            void *workspace_dev, size_t workspace_bytes) {
    TTL_REQUIRE(shift_dev, TTL_ERR_INVALID, "ttl_matmul_q8_0_shifted: null shifts");
    return matmul_q8_0(ctx, w, bias_dev, x_dev, shift_dev, tokens, residual_dev, out_dev, workspace_dev,
                       workspace_bytes, "ttl_matmul_q8_0_shifted");
}

}  // extern "C"
