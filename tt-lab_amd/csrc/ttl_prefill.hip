// Batched (prefill) MXFP4 expert GEMMs on MFMA.
//
// Two entry points share the kernels:
//  - ttl_matmul_mxfp4_selected: the selected-token matmul of one expert,
//    matmul_add_mxfp4_selected_transposed (tensor.cpp:306-495);
//  - ttl_moe_prefill_experts: the expert half of GptOssModel::moe_batch
//    (model.cpp:378-460) for a batch of tokens whose routing is given.
//
// Numerics.  v_mfma_f32_16x16x32_bf16 accumulates in f32, and every product it
// forms is exact:
//  - a weight E2M1 x 2^(e-127) has at most two significant bits, so it is a bf16
//    exactly for E8M0 e in 1..254; v_cvt_scalef32_pk_bf16_fp4 decodes it in registers;
//  - an f32 activation is split into three bf16 planes whose sum is the value
//    exactly (mf::split_planes); a bf16 activation is one plane.
// The MFMA therefore sums the reference's exact products in f32, starting from the
// bias as the reference does (tensor.cpp:455-462), in a different order: results
// agree to f32 rounding, not bit for bit.
//
// Data flow of ttl_moe_prefill_experts (S = count * used (token, rank) pairs):
//  1. plan_kernel (one workgroup): buckets the pairs by expert in the reference's
//     order (model.cpp:380-394: expert-major, then token, then rank); a pair's
//     position in that order is its slot.  Each expert's bucket is cut into tiles
//     of 64 slots.
//  2. gather_kernel: the tokens of every tile as MFMA B fragments (bf16 planes).
//  3. gateup_kernel: per (tile, 128 rows) the gate and up GEMMs, the clamped SwiGLU
//     in registers, and the hidden written straight into the down GEMM's B
//     fragments (a lane's D rows 4g..4g+3 of the two 16-row tiles of one 32-row
//     block are exactly the 8 values of the down fragment for K step g).
//  4. matmul_kernel: the down GEMM per (tile, 192 rows), f32 output per slot.
//  5. combine_kernel: out[token] = sum over the token's slots in expert order of
//     weight * down, unfused, from 0 (model.cpp:380,450-459).
#include "ttl_mfma.hpp"
#include "ttl_moe_math.hpp"

#include <cmath>

namespace {

using mf::bf16x8;
using mf::f32x4;

constexpr uint32_t kMaxExperts = 256;
constexpr uint32_t kMaxUsed = 16;
constexpr uint32_t kPlanThreads = 1024;
constexpr uint32_t kMaxEntries = 1u << 22;  // count * used

// gate/up: 4 waves x 32 rows (two 16-row tiles of gate and of up per wave); two
// workgroups share a CU, one wave of each per SIMD
constexpr int kGuWaves = 4;
constexpr int kGuRows = kGuWaves * 32;
constexpr int kGuCodeBuffers = 4;  // weight codes are requested this many quads minus one ahead
// matmul (down): 4 waves x 48 rows (three 16-row tiles per wave)
constexpr int kMmWaves = 4;
constexpr int kMmTiles = 3;
constexpr int kMmRows = kMmWaves * kMmTiles * 16;

// Hidden planes between gate/up and down: three, exact (the hidden is f32).
constexpr int kHiddenPlanes = 3;

// A tile holding at most kNarrowSlots slots (the remainder of an expert's bucket) is
// "narrow": its GEMMs run on the first kNarrowCols column tiles only (a branch of the
// same launch), so a bucket of 70 slots costs 64 + 32 columns instead of 64 + 64.
constexpr int kNarrowCols = 2;
constexpr uint32_t kNarrowSlots = kNarrowCols * 16;

// ---- the plan ------------------------------------------------------------------

struct PlanHeader {
    uint32_t tiles;    // token tiles in use
    uint32_t invalid;  // pairs whose expert index was out of range
    uint32_t wide;     // tiles [0, wide) hold more than kNarrowSlots slots, [wide, tiles) at most that
    uint32_t pad[61];
};

// Device pointers into the caller's workspace.
struct Plan {
    PlanHeader *header;
    uint32_t *tile_expert;  // [tmax]
    uint32_t *tile_first;   // [tmax] first slot
    uint32_t *tile_count;   // [tmax] slots in the tile (1..64)
    uint32_t *slot_token;   // [S]
    float *slot_weight;     // [S]
    int32_t *pair_slot;     // [S] slot of pair (token, rank) = token*used + rank, -1 if invalid
    uint8_t *xb;            // [tmax][x planes][plane_bytes]
    uint8_t *hb;            // [tmax][hidden planes][plane_bytes]
    float *down;            // [S][rows]
    int32_t *token_shift;   // [tokens] k of each token row (f16 token planes hold x 2^k)
    int32_t *tile_shift;    // [tmax][64] k of each tile column (0 past the tile's slots)
};

struct Layout {
    size_t header, tile_expert, tile_first, tile_count, slot_token, slot_weight, pair_slot, xb, hb, down,
        token_shift, tile_shift, total;
    uint32_t tmax;
};

size_t align256(size_t v) {
    return (v + 255) & ~size_t(255);
}

// Upper bound on the tiles: sum_e ceil(c_e / T) <= (S + (T - 1) * nonempty) / T for
// tiles of T = mf::tile_slots slots.
uint32_t max_tiles(uint32_t pairs, uint32_t experts) {
    const uint32_t nonempty = pairs < experts ? pairs : experts;
    return uint32_t((uint64_t(pairs) + uint64_t(mf::tile_slots - 1) * nonempty) / mf::tile_slots) + 1;
}

// tokens > 0: room for the token and tile shifts of f16 token planes.
Layout make_layout(uint32_t pairs, uint32_t experts, int x_planes, bool with_hidden, uint32_t rows,
                   uint32_t tokens = 0) {
    Layout L{};
    L.tmax = max_tiles(pairs, experts);
    size_t o = 0;
    L.header = o;
    o = align256(o + sizeof(PlanHeader));
    L.tile_expert = o;
    o = align256(o + 4ull * L.tmax);
    L.tile_first = o;
    o = align256(o + 4ull * L.tmax);
    L.tile_count = o;
    o = align256(o + 4ull * L.tmax);
    L.slot_token = o;
    o = align256(o + 4ull * pairs);
    L.slot_weight = o;
    o = align256(o + 4ull * pairs);
    L.pair_slot = o;
    o = align256(o + 4ull * pairs);
    L.xb = o;
    o = align256(o + size_t(L.tmax) * x_planes * mf::plane_bytes);
    L.hb = o;
    if (with_hidden) {
        o = align256(o + size_t(L.tmax) * kHiddenPlanes * mf::plane_bytes);
    }
    L.down = o;
    if (with_hidden) {
        o = align256(o + 4ull * pairs * rows);
    }
    L.token_shift = o;
    L.tile_shift = o;
    if (tokens > 0) {
        o = align256(o + 4ull * tokens);
        L.tile_shift = o;
        o = align256(o + 4ull * L.tmax * mf::tile_slots);
    }
    L.total = o;
    return L;
}

Plan plan_at(void *workspace, const Layout &L) {
    uint8_t *w = static_cast<uint8_t *>(workspace);
    Plan p;
    p.header = reinterpret_cast<PlanHeader *>(w + L.header);
    p.tile_expert = reinterpret_cast<uint32_t *>(w + L.tile_expert);
    p.tile_first = reinterpret_cast<uint32_t *>(w + L.tile_first);
    p.tile_count = reinterpret_cast<uint32_t *>(w + L.tile_count);
    p.slot_token = reinterpret_cast<uint32_t *>(w + L.slot_token);
    p.slot_weight = reinterpret_cast<float *>(w + L.slot_weight);
    p.pair_slot = reinterpret_cast<int32_t *>(w + L.pair_slot);
    p.xb = w + L.xb;
    p.hb = w + L.hb;
    p.down = reinterpret_cast<float *>(w + L.down);
    p.token_shift = reinterpret_cast<int32_t *>(w + L.token_shift);
    p.tile_shift = reinterpret_cast<int32_t *>(w + L.tile_shift);
    return p;
}

// Exclusive prefix sum over the 64 lanes of a wave (all lanes active).
__device__ inline uint32_t wave_exclusive_sum(uint32_t v, uint32_t lane) {
    uint32_t x = v;
#pragma unroll
    for (uint32_t d = 1; d < 64; d <<= 1) {
        const uint32_t y = __shfl_up(x, d);
        x += lane >= d ? y : 0u;
    }
    return x - v;
}

// Buckets the (token, rank) pairs by expert in the reference's order and cuts the
// buckets into 64-slot tiles.  One workgroup of 1024 threads; pairs are taken in
// rounds of 1024 in pair order, and a pair's slot is its expert's base plus the
// number of earlier pairs with the same expert.  Each thread requests the indices and
// weights of its first kPlanHeld rounds at once, at the start (a 512-token batch of
// top-4 is two rounds), so the kernel waits for global memory once instead of once
// per pass; later rounds load theirs as they come.
constexpr uint32_t kPlanHeld = 2;
constexpr uint32_t kPlanPerLane = kMaxExperts / 64;  // experts per lane in the bucket scan

__global__ __launch_bounds__(kPlanThreads) void plan_kernel(const int32_t *__restrict__ indices,
                                                            const float *__restrict__ weights, uint32_t pairs,
                                                            uint32_t used, uint32_t experts, Plan plan) {
    __shared__ uint32_t count[kMaxExperts], base[kMaxExperts], running[kMaxExperts], narrow_of[kMaxExperts];
    __shared__ uint32_t wide_total;
    __shared__ uint32_t wave_count[kPlanThreads / 64][kMaxExperts];
    __shared__ uint32_t invalid;
    const uint32_t t = threadIdx.x, lane = t % 64, wave = t / 64;
    const uint32_t rounds = (pairs + kPlanThreads - 1) / kPlanThreads;
    // expert of pair j, -1 for an index out of range or past the pairs
    auto expert_of = [&](int32_t e, uint32_t j) __attribute__((always_inline)) {
        return j < pairs && e >= 0 && uint32_t(e) < experts ? e : -1;
    };
    int32_t held_e[kPlanHeld];
    float held_w[kPlanHeld];
#pragma unroll
    for (uint32_t k = 0; k < kPlanHeld; ++k) {
        // unconditional (clamped) requests; pairs == 0 never launches
        const uint32_t j = min(t + k * kPlanThreads, pairs - 1);
        held_e[k] = indices[j];
        held_w[k] = weights[j];
    }
    for (uint32_t e = t; e < kMaxExperts; e += kPlanThreads) {
        count[e] = 0;
    }
    if (t == 0) {
        invalid = 0;
    }
    __syncthreads();
    auto count_pair = [&](int32_t raw, uint32_t j) __attribute__((always_inline)) {
        const int32_t e = expert_of(raw, j);
        if (e >= 0) {
            atomicAdd(&count[e], 1u);
        } else if (j < pairs) {
            atomicAdd(&invalid, 1u);
        }
    };
    // the held rounds with constant indices (a run-time index would put them in scratch)
#pragma unroll
    for (uint32_t k = 0; k < kPlanHeld; ++k) {
        count_pair(held_e[k], k * kPlanThreads + t);
    }
    for (uint32_t r = kPlanHeld; r < rounds; ++r) {
        const uint32_t j = r * kPlanThreads + t;
        count_pair(indices[min(j, pairs - 1)], j);
    }
    __syncthreads();
    if (wave == 0) {
        // wide tiles in expert order first, then the narrow ones (an expert's last tile
        // when it holds at most kNarrowSlots slots), also in expert order: lane l takes
        // experts kPlanPerLane l .. + kPlanPerLane - 1, and one prefix sum per quantity
        // places them after the lanes before
        uint32_t c[kPlanPerLane], slots = 0, wide = 0, narrow = 0;
#pragma unroll
        for (uint32_t k = 0; k < kPlanPerLane; ++k) {
            const uint32_t e = lane * kPlanPerLane + k;
            c[k] = e < experts ? count[e] : 0u;
            const uint32_t tiles = (c[k] + mf::tile_slots - 1) / mf::tile_slots;
            const bool last_narrow = tiles > 0 && c[k] - (tiles - 1) * mf::tile_slots <= kNarrowSlots;
            slots += c[k];
            wide += tiles - (last_narrow ? 1u : 0u);
            narrow += last_narrow ? 1u : 0u;
        }
        uint32_t s0 = wave_exclusive_sum(slots, lane), w0 = wave_exclusive_sum(wide, lane),
                 n0 = wave_exclusive_sum(narrow, lane);
#pragma unroll
        for (uint32_t k = 0; k < kPlanPerLane; ++k) {
            const uint32_t e = lane * kPlanPerLane + k;
            const uint32_t tiles = (c[k] + mf::tile_slots - 1) / mf::tile_slots;
            const bool last_narrow = tiles > 0 && c[k] - (tiles - 1) * mf::tile_slots <= kNarrowSlots;
            if (e < experts) {
                base[e] = s0;
                running[e] = w0;  // first wide tile of expert e (reset below)
                narrow_of[e] = last_narrow ? n0 : ~0u;
            }
            s0 += c[k];
            w0 += tiles - (last_narrow ? 1u : 0u);
            n0 += last_narrow ? 1u : 0u;
        }
        if (lane == 63) {
            wide_total = w0;
            plan.header->tiles = w0 + n0;
            plan.header->wide = w0;
            plan.header->invalid = invalid;
        }
    }
    __syncthreads();
    for (uint32_t e = t; e < experts; e += kPlanThreads) {
        const uint32_t n = count[e];
        for (uint32_t j = 0; j * mf::tile_slots < n; ++j) {
            const bool last = (j + 1) * mf::tile_slots >= n;
            const uint32_t tile = last && narrow_of[e] != ~0u ? wide_total + narrow_of[e] : running[e] + j;
            plan.tile_expert[tile] = e;
            plan.tile_first[tile] = base[e] + j * mf::tile_slots;
            plan.tile_count[tile] = min(uint32_t(mf::tile_slots), n - j * mf::tile_slots);
        }
    }
    __syncthreads();
    for (uint32_t e = t; e < kMaxExperts; e += kPlanThreads) {
        running[e] = 0;
    }
    // one round of 1024 pairs (uniform across the workgroup: its barriers are reached by all)
    auto place_round = [&](uint32_t r, int32_t raw, float wj) __attribute__((always_inline)) {
        for (uint32_t e = t; e < (kPlanThreads / 64) * kMaxExperts; e += kPlanThreads) {
            (&wave_count[0][0])[e] = 0;
        }
        __syncthreads();
        const uint32_t j = r * kPlanThreads + t;
        const int32_t ej = expert_of(raw, j);
        const bool valid = ej >= 0;
        // the lanes of this wave with the same expert: one ballot per bit of the expert
        // index (a lane matches where every bit agrees); rank = earlier lanes among them,
        // and the lowest of them records the wave's count for the expert
        uint64_t same = __ballot(valid);
        for (uint32_t bit = 0; (1u << bit) < experts; ++bit) {
            const bool one = valid && ((uint32_t(ej) >> bit) & 1u);
            const uint64_t ones = __ballot(one);
            same &= one ? ones : ~ones;
        }
        const uint32_t rank = uint32_t(__popcll(same & ((1ull << lane) - 1ull)));
        if (valid && rank == 0) {
            wave_count[wave][ej] = uint32_t(__popcll(same));
        }
        __syncthreads();
        if (j < pairs) {
            if (valid) {
                uint32_t slot = base[ej] + running[ej] + rank;
#pragma unroll
                for (uint32_t w = 0; w < kPlanThreads / 64; ++w) {
                    slot += w < wave ? wave_count[w][ej] : 0u;
                }
                plan.slot_token[slot] = j / used;
                plan.slot_weight[slot] = wj;
                plan.pair_slot[j] = int32_t(slot);
            } else {
                plan.pair_slot[j] = -1;
            }
        }
        __syncthreads();
        for (uint32_t e = t; e < experts; e += kPlanThreads) {
            uint32_t add = 0;
            for (uint32_t w = 0; w < kPlanThreads / 64; ++w) {
                add += wave_count[w][e];
            }
            running[e] += add;
        }
        __syncthreads();
    };
#pragma unroll
    for (uint32_t k = 0; k < kPlanHeld; ++k) {
        if (k < rounds) {
            place_round(k, held_e[k], held_w[k]);
        }
    }
    for (uint32_t r = kPlanHeld; r < rounds; ++r) {
        const uint32_t jc = min(r * kPlanThreads + t, pairs - 1);
        place_round(r, indices[jc], weights[jc]);
    }
}

// The plan of one selected-token matmul: one expert, slot s = token tokens[s].
__global__ void plan_selected_kernel(const int32_t *__restrict__ tokens, uint32_t count, uint32_t expert,
                                     Plan plan) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t tiles = (count + mf::tile_slots - 1) / mf::tile_slots;
    if (i == 0) {
        plan.header->tiles = tiles;
        plan.header->wide = tiles;  // one launch over every tile
        plan.header->invalid = 0;
    }
    if (i < tiles) {
        plan.tile_expert[i] = expert;
        plan.tile_first[i] = i * mf::tile_slots;
        plan.tile_count[i] = min(uint32_t(mf::tile_slots), count - i * mf::tile_slots);
    }
    if (i < count) {
        plan.slot_token[i] = uint32_t(tokens[i]);  // range-checked where it is used
        plan.slot_weight[i] = 1.0f;
        plan.pair_slot[i] = int32_t(i);
    }
}

// ---- activation fragments ------------------------------------------------------------

// Row shifts (ttl::launch_row_shifts): one wave per row, four rows per workgroup; each
// lane requests its (at most 16) float4 of the row at once, clamped to the row's last
// (a repeated value leaves the maximum unchanged).
constexpr uint32_t kShiftRowsPerBlock = 4;
constexpr uint32_t kShiftMaxCols = 4096;

__global__ __launch_bounds__(kShiftRowsPerBlock * 64) void row_shift_kernel(const float *__restrict__ x,
                                                                            uint32_t stride, uint32_t rows,
                                                                            uint32_t cols,
                                                                            int32_t *__restrict__ shift) {
    const uint32_t row = blockIdx.x * kShiftRowsPerBlock + threadIdx.x / 64, lane = threadIdx.x % 64;
    if (row >= rows) {
        return;
    }
    const float4 *p = reinterpret_cast<const float4 *>(x + size_t(row) * stride);
    const uint32_t n4 = cols / 4;
    constexpr int kPer = kShiftMaxCols / 4 / 64;
    float4 v[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        v[j] = p[min(lane + 64u * j, n4 - 1)];
    }
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        m = mf::finite_max(mf::finite_max(mf::finite_max(mf::finite_max(m, v[j].x), v[j].y), v[j].z), v[j].w);
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        m = __builtin_fmaxf(m, __shfl_xor(m, d));
    }
    if (lane == 0) {
        shift[row] = mf::row_shift(m);
    }
}

// One workgroup per (quad, token tile); thread (column tile, lane) takes slot
// 16 ct + lane % 16 and K-block 4 quad + lane / 16, i.e. the 8 activations of that B
// fragment lane in each of the quad's four K steps: one 128-byte run of the row (f32;
// 64 bytes for bf16), converted to P bf16 planes per step.  The tile's metadata and
// the early exit are requested together, then the slot's token, then its row
// (unconditional requests at clamped addresses, masked after).  Slots past the tile's
// count, and blocks 90/91, are zero; a token out of range is NaN.  F16X (f32 rows, P = 2):
// the planes are two f16 of x 2^k with the token's k from plan.token_shift, and the quad-0
// workgroups record each column's k in plan.tile_shift (0 for an empty or NaN column).
template <bool BF16_IN, int P, bool F16X = false>
__global__ __launch_bounds__(mf::col_tiles * 64) void gather_kernel(const void *__restrict__ x, uint32_t x_stride,
                                                                    uint32_t x_rows, Plan plan) {
    static_assert(!F16X || (P == 2 && !BF16_IN), "f16 token planes are two, from f32 rows");
    const uint32_t tile = blockIdx.y, quad = blockIdx.x;
    // (tile < the layout's tmax: its metadata words exist, stale past the plan's tiles)
    const uint32_t tiles = plan.header->tiles, cnt = plan.tile_count[tile], first = plan.tile_first[tile];
    if (tile >= tiles) {
        return;
    }
    const uint32_t ct = threadIdx.x / 64, lane = threadIdx.x % 64;
    const uint32_t n = ct * 16 + lane % 16;
    const uint32_t block = quad * 4 + lane / 16;
    const bool block_ok = block < uint32_t(mx::blocks);
    const uint32_t token = plan.slot_token[first + min(n, cnt - 1)];
    const bool live = n < cnt && block_ok;
    const bool token_ok = token < x_rows;
    const size_t base = size_t(token_ok ? token : 0u) * x_stride + size_t(block_ok ? block : 0u) * 32;
    // the block's 32 activations as f32
    float e[32];
    if (BF16_IN) {
        const uint4 *src = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(x) + base);
        uint4 w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            w[k] = src[k];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t ww[4] = {w[k].x, w[k].y, w[k].z, w[k].w};
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                e[8 * k + 2 * h] = __uint_as_float(ww[h] << 16);
                e[8 * k + 2 * h + 1] = __uint_as_float(ww[h] & 0xffff0000u);
            }
        }
    } else {
        const float4 *src = reinterpret_cast<const float4 *>(static_cast<const float *>(x) + base);
        float4 w[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            w[k] = src[k];
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            e[4 * k] = w[k].x;
            e[4 * k + 1] = w[k].y;
            e[4 * k + 2] = w[k].z;
            e[4 * k + 3] = w[k].w;
        }
    }
    const float fill = (live && !token_ok) ? __builtin_nanf("") : 0.0f;
    const bool keep = live && token_ok;
    int k = 0;
    if constexpr (F16X) {
        const int kt = plan.token_shift[token_ok ? token : 0u];
        k = keep ? kt : 0;
        if (quad == 0 && lane < 16) {
            plan.tile_shift[size_t(tile) * mf::tile_slots + n] = k;
        }
    }
    uint8_t *dst = plan.xb + size_t(tile) * P * mf::plane_bytes + size_t(ct) * mf::frag_bytes + lane * 16;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        // step s of the quad: elements 4s..4s+3 and 16+4s..16+4s+3, interleaved
        float v[8];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[2 * k] = keep ? e[4 * s + k] : fill;
            v[2 * k + 1] = keep ? e[16 + 4 * s + k] : fill;
        }
        uint4 out[P];
        if constexpr (F16X) {
            mf::split_f16x2(v, k, out);
        } else {
            mf::split_planes<P>(v, out);
        }
        const size_t step = size_t(quad) * 4 + size_t(s);
#pragma unroll
        for (int p = 0; p < P; ++p) {
            *reinterpret_cast<uint4 *>(dst + size_t(p) * mf::plane_bytes + step * mf::col_tiles * mf::frag_bytes) =
                out[p];
        }
    }
}

// ---- the MFMA main loop ----------------------------------------------------------------

// K steps per LDS stage for P activation planes: a stage holds P * steps * 4
// fragments (16 KiB for one plane, 24 KiB for three).
template <int P>
struct StageShape {
    static constexpr int steps = P == 1 ? 4 : 2;
    static constexpr int count = mf::steps / steps;
    static constexpr int frags = P * steps * mf::col_tiles;
    static constexpr int chunks = frags * 64;  // 16-byte pieces
    static_assert(mf::steps % steps == 0, "stages must divide the K steps");
};

// Copies stage `j` of a token tile's fragments (P planes) between global memory
// and LDS through registers; LDS order is [plane][step][column tile][lane].  Every
// thread moves `per` pieces with no condition (a branch around a load makes the
// compiler wait for it at once): pieces past the stage re-read its last piece and
// land in the LDS buffer's padding.
template <int P, int THREADS>
struct Stager {
    using SS = StageShape<P>;
    static constexpr int per = (SS::chunks + THREADS - 1) / THREADS;
    static constexpr int lds_chunks = per * THREADS;  // LDS buffer size in pieces
    mf::u32x4 r[per];

    __device__ inline void load(const uint8_t *__restrict__ tile_frags, int j, uint32_t t) {
#pragma unroll
        for (int k = 0; k < per; ++k) {
            const uint32_t c = min(t + uint32_t(k) * THREADS, uint32_t(SS::chunks - 1));
            const uint32_t plane = c / (SS::steps * mf::col_tiles * 64);
            const uint32_t within = c % (SS::steps * mf::col_tiles * 64);
            r[k] = *reinterpret_cast<const mf::u32x4 *>(tile_frags + size_t(plane) * mf::plane_bytes +
                                                    size_t(j) * SS::steps * mf::col_tiles * mf::frag_bytes +
                                                    size_t(within) * 16);
        }
    }
    __device__ inline void store(mf::u32x4 *lds, uint32_t t) const {
#pragma unroll
        for (int k = 0; k < per; ++k) {
            lds[t + uint32_t(k) * THREADS] = r[k];
        }
    }
};

// One wave's A operand: NT 16-row tiles of repacked MXFP4 (ttl_internal.hpp), the
// codes of one quad (4 K steps) per tile and the lane's 24 scale bytes per tile.
template <int NT>
struct AOperand {
    const uint4 *codes[NT];  // tile base + lane row
    uint32_t sw[NT][6];

    __device__ inline void init(const uint8_t *__restrict__ codes_base, const uint8_t *__restrict__ scales_base,
                                const size_t (&tile_index)[NT], uint32_t lane) {
#pragma unroll
        for (int a = 0; a < NT; ++a) {
            codes[a] = reinterpret_cast<const uint4 *>(codes_base) + tile_index[a] * mx::blocks * mx::tile_rows +
                       lane % mx::tile_rows;
            const uint2 *rec = reinterpret_cast<const uint2 *>(scales_base + tile_index[a] * mx::tile_scale_bytes +
                                                               size_t(lane) * mx::scale_pad);
            const uint2 s01 = rec[0], s23 = rec[1], s45 = rec[2];
            sw[a][0] = s01.x;
            sw[a][1] = s01.y;
            sw[a][2] = s23.x;
            sw[a][3] = s23.y;
            sw[a][4] = s45.x;
            sw[a][5] = s45.y;
        }
    }
    // Codes of quad i (blocks 4i..4i+3; past block 89 the lane re-reads block 89,
    // whose activations there are zero and whose scale byte is the padding 127).
    __device__ inline void load(int i, uint32_t lane, uint4 (&q)[NT]) const {
        const uint32_t block = min(uint32_t(4 * i) + lane / mx::tile_rows, uint32_t(mx::blocks - 1));
#pragma unroll
        for (int a = 0; a < NT; ++a) {
            q[a] = ttl::load_stream(codes[a] + size_t(block) * mx::tile_rows);
        }
    }
    // The same for tile a alone.
    __device__ inline uint4 load_one(int i, uint32_t lane, int a) const {
        const uint32_t block = min(uint32_t(4 * i) + lane / mx::tile_rows, uint32_t(mx::blocks - 1));
        return ttl::load_stream(codes[a] + size_t(block) * mx::tile_rows);
    }
    // Scale of tile a for the current quad; next_quad() moves every record on by
    // one byte, so the indices stay static.
    __device__ inline float scale(int a) const {
        return mf::e8m0_scale(sw[a][0] & 0xffu);
    }
    __device__ inline uint32_t scale_byte(int a) const {
        return sw[a][0] & 0xffu;
    }
    __device__ inline void next_quad() {
#pragma unroll
        for (int a = 0; a < NT; ++a) {
#pragma unroll
            for (int k = 0; k < 5; ++k) {
                sw[a][k] = (sw[a][k] >> 8) | (sw[a][k + 1] << 24);
            }
            sw[a][5] >>= 8;
        }
    }
};

// The MFMAs of quad i (K steps 4i..4i+3) for M 16-row A tiles and P activation
// planes: acc[m][c] += A_m * B(p, c) in the order c, then p, per step.  B
// fragments are read LOOK fragments before their MFMAs, within a stage (the
// next stage is readable only after the barrier that ends this one), so the wave
// waits for LDS about once per stage rather than once per fragment.
// decode(s, w) fills the M A fragments of step s of the quad; stage_end(stage)
// runs after the last MFMA of each stage (publishes the next one).  Only the first
// NC column tiles are multiplied (narrow tiles leave the others unread).
template <int P, int M, int LOOK, int NC, class V = bf16x8, class Decode, class StageEnd>
__device__ __attribute__((always_inline)) inline void quad_mfma(const mf::u32x4 *buf0, const mf::u32x4 *buf1,
                                                                int i, uint32_t lane, Decode &&decode,
                                                                StageEnd &&stage_end, f32x4 (&acc)[M][NC]) {
    using SS = StageShape<P>;
    static_assert(NC >= 1 && NC <= mf::col_tiles, "column tiles");
    constexpr int FPS = P * NC;  // fragments per K step
    constexpr int SF = SS::steps * FPS;     // fragments per stage
    constexpr int D = LOOK < SF ? LOOK : SF;
#pragma unroll
    for (int q = 0; q < 4 / SS::steps; ++q) {
        const int stage = (4 * i) / SS::steps + q;
        const mf::u32x4 *buf = (stage % 2) ? buf1 : buf0;
        auto frag = [&](int f) __attribute__((always_inline)) {
            const int ls = f / FPS, c = (f % FPS) / P, p = f % P;
            return __builtin_bit_cast(V, buf[((p * SS::steps + ls) * mf::col_tiles + c) * 64 + lane]);
        };
        V ring[D];
#pragma unroll
        for (int d = 0; d < D; ++d) {
            ring[d] = frag(d);
        }
        V w[M];
#pragma unroll
        for (int f = 0; f < SF; ++f) {
            const V b = ring[f % D];
            if (f + D < SF) {
                ring[f % D] = frag(f + D);
            }
            if (f % FPS == 0) {
                decode(q * SS::steps + f / FPS, w);
            }
            const int c = (f % FPS) / P;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                acc[m][c] = mf::mfma(w[m], b, acc[m][c]);
            }
        }
        stage_end(stage);
    }
}

// Quads 0..22 with NB code buffers rotating under static indices: quad i's codes
// are requested NB - 1 quads before they are used (requests past quad 22 repeat
// it).  The caller has requested quads 0..NB-2 into buffers 0..NB-2.  Each request
// is pinned before the quad's instructions (sched_barrier), and so are the stage
// requests at every stage end: left to the scheduler, requests sank to just before
// their first use and the wave waited for them there.
template <int NB, int M, class Load, class Compute>
__device__ __attribute__((always_inline)) inline void rotate_quads(uint4 (&qa)[NB][M], Load &&load,
                                                                   Compute &&compute) {
    for (int i = 0; i < mf::quads; i += NB) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (i + b < mf::quads) {
                load(min(i + b + NB - 1, mf::quads - 1), qa[(b + NB - 1) % NB]);
                __builtin_amdgcn_sched_barrier(0);
                compute(i + b, qa[b]);
            }
        }
    }
}

// ---- gate/up + SwiGLU -------------------------------------------------------------------

struct GateUpArgs {
    const uint8_t *gate_codes, *gate_scales, *up_codes, *up_scales;
    const float *gate_bias, *up_bias;  // [experts][rows] or null
    uint32_t rows, tiles_per_expert;
    Plan plan;
};

// Workgroup -> (token tile, row group).  Workgroups are dispatched round-robin
// over the chip's 8 XCDs (each with its own L2), so consecutive logical indices
// are taken from the same XCD: all row groups of one token tile then read its
// activation fragments through one L2.  Workgroups past the tiles in use return.
__device__ inline bool tile_in_range(uint32_t tiles, uint32_t &tile, uint32_t &row_group) {
    const uint32_t groups = gridDim.x;
    const uint32_t id = blockIdx.y * groups + blockIdx.x;
    const uint32_t active = tiles * groups;
    if (id >= active) {
        return false;
    }
    const uint32_t logical = active % 8 == 0 ? (id % 8) * (active / 8) + id / 8 : id;
    tile = logical / groups;
    row_group = logical % groups;
    return true;
}

// One launch covers every tile of the plan: the wide tiles [0, wide) run with all
// mf::col_tiles column tiles, the narrow ones [wide, tiles) with kNarrowCols (the
// workgroup's branch is uniform, so the barriers inside are reached by all its waves).
__device__ inline bool tile_of_workgroup(const PlanHeader *header, uint32_t &tile, uint32_t &row_group,
                                         bool &narrow) {
    if (!tile_in_range(header->tiles, tile, row_group)) {
        return false;
    }
    narrow = tile >= header->wide;
    return true;
}

// Accumulators: [matrix (gate 0/1, up 2/3)][column tile]; NC column tiles (the plan's
// wide tiles with all of them, or its narrow ones with kNarrowCols).
// F16H: the hidden as two f16 planes of h x 2^kHiddenF16Shift (for the f16 down GEMM),
// else three exact bf16 planes.  VX: the token operand, bf16x8 (PX exact planes; the
// accumulators start at the bias) or f16x8 (two planes of x 2^k per column, k from
// plan.tile_shift; the weights decoded to f16): then the accumulators start at zero, and
// the sums are scaled back by 2^-k and the bias added before the SwiGLU.
template <int PX, int NC, bool F16H, class VX>
__device__ __attribute__((always_inline)) inline void gateup_tile(
    const GateUpArgs &a, uint32_t tile, uint32_t row_group,
    mf::u32x4 (*lds)[Stager<PX, kGuWaves * 64>::lds_chunks]) {
    constexpr bool XS = __is_same(VX, mf::f16x8);
    static_assert(!XS || PX == 2, "f16 token operands are two planes");
    using SS = StageShape<PX>;
    constexpr int kThreads = kGuWaves * 64;
    const uint32_t t = threadIdx.x, wave = t / 64, lane = t % 64;
    const uint32_t expert = a.plan.tile_expert[tile];
    const uint32_t row0 = row_group * kGuRows + wave * 32;  // this wave's 32 rows (one down K block)
    // waves past the last row only help stage; they read the first wave's rows
    // (L2 hits) so that every wave runs the same code
    const bool rows_ok = row0 < a.rows;
    const uint32_t row_base = rows_ok ? row0 : row_group * kGuRows;
    const size_t tile0 = size_t(expert) * a.tiles_per_expert + row_base / 16;
    const uint8_t *frags = a.plan.xb + size_t(tile) * PX * mf::plane_bytes;

    AOperand<2> ga, ua;
    const size_t ti[2] = {tile0, tile0 + 1};
    ga.init(a.gate_codes, a.gate_scales, ti, lane);
    ua.init(a.up_codes, a.up_scales, ti, lane);

    // the bias of the lane's D rows 4g..4g+3 of matrix m (gate 0/1, up 2/3)
    auto bias_of = [&](int m) __attribute__((always_inline)) {
        const float *bias = m < 2 ? a.gate_bias : a.up_bias;
        f32x4 b = {0.f, 0.f, 0.f, 0.f};
        if (bias) {
            const float4 v = *reinterpret_cast<const float4 *>(bias + size_t(expert) * a.rows + row_base +
                                                               16 * (m % 2) + 4 * (lane / 16));
            b = f32x4{v.x, v.y, v.z, v.w};
        }
        return b;
    };
    f32x4 acc[4][NC];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        f32x4 b;
        if constexpr (XS) {
            // a zero the compiler cannot see: starting the MFMA chains from a known
            // zero made it keep extra registers through the loop (34 spilled)
            float z;
            asm volatile("v_mov_b32 %0, 0" : "=v"(z));
            b = f32x4{z, z, z, z};
        } else {
            b = bias_of(m);
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            acc[m][c] = b;
        }
    }

    Stager<PX, kThreads> st;
    st.load(frags, 0, t);
    // three planes leave room for one code buffer less (the fourth spilled)
    constexpr int NB = PX == 3 ? 3 : kGuCodeBuffers;
    uint4 qa[NB][4];  // codes of the quads in flight: [buffer][gate0, gate1, up0, up1]
    auto load_quad = [&](int i, uint4(&q)[4]) __attribute__((always_inline)) {
        uint4 g2[2], u2[2];
        ga.load(i, lane, g2);
        ua.load(i, lane, u2);
        q[0] = g2[0];
        q[1] = g2[1];
        q[2] = u2[0];
        q[3] = u2[1];
    };
#pragma unroll
    for (int b = 0; b < NB - 1; ++b) {
        load_quad(b, qa[b]);
    }
    st.store(lds[0], t);
    __syncthreads();
    if (SS::count > 1) {
        st.load(frags, 1, t);
    }

    auto stage_end = [&](int stage) __attribute__((always_inline)) {
        // end of stage: publish the next stage, fetch the one after
        if (stage + 1 < SS::count) {
            st.store(lds[(stage + 1) % 2], t);
        }
        __syncthreads();
        if (stage + 2 < SS::count) {
            st.load(frags, stage + 2, t);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    auto compute_quad = [&](int i, const uint4(&q)[4]) __attribute__((always_inline)) {
        float sc[4];
        sc[0] = ga.scale(0);
        sc[1] = ga.scale(1);
        sc[2] = ua.scale(0);
        sc[3] = ua.scale(1);
        ga.next_quad();
        ua.next_quad();
        auto decode = [&](int s, VX(&w)[4]) __attribute__((always_inline)) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const uint32_t word = s == 0 ? q[m].x : (s == 1 ? q[m].y : (s == 2 ? q[m].z : q[m].w));
                w[m] = mf::decode_as<VX>(word, sc[m]);
            }
        };
        // B fragments four ahead of their MFMAs for one plane and for three (with three
        // planes this fits the 256 registers of two waves per SIMD without spilling)
        quad_mfma<PX, 4, 4, NC, VX>(lds[0], lds[1], i, lane, decode, stage_end, acc);
    };

    rotate_quads(qa, load_quad, compute_quad);
    if (!rows_ok) {
        return;
    }

    // SwiGLU and the hidden as down-GEMM B fragments: this wave's 32 rows are down K
    // block beta; lane (n, g) holds rows 4g..4g+3 of both 16-row halves, i.e. the
    // 8 values of K step g of that block for token n.
    const uint32_t beta = row0 / 32, quad = beta / 4, gb = beta % 4;
    const uint32_t g = lane / 16, n16 = lane % 16;
    uint8_t *hb = a.plan.hb + size_t(tile) * kHiddenPlanes * mf::plane_bytes;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        if constexpr (XS) {
            // the column's sums scaled back, then the bias
            const int k = a.plan.tile_shift[size_t(tile) * mf::tile_slots + c * 16 + n16];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const f32x4 b = bias_of(m);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    acc[m][c][i] = b[i] + __builtin_amdgcn_ldexpf(acc[m][c][i], -k);
                }
            }
        }
        float h[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            h[2 * i] = moe_math::clamped_swiglu(acc[0][c][i], acc[2][c][i]);
            h[2 * i + 1] = moe_math::clamped_swiglu(acc[1][c][i], acc[3][c][i]);
        }
        constexpr int HP = F16H ? 2 : kHiddenPlanes;
        uint4 planes[HP];
        if constexpr (F16H) {
            mf::split_f16x2(h, mf::kHiddenF16Shift, planes);
        } else {
            mf::split_planes<HP>(h, planes);
        }
        const size_t off = ((size_t(quad) * 4 + g) * mf::col_tiles + c) * mf::frag_bytes + (gb * 16 + n16) * 16;
#pragma unroll
        for (int p = 0; p < HP; ++p) {
            *reinterpret_cast<uint4 *>(hb + size_t(p) * mf::plane_bytes + off) = planes[p];
        }
        // blocks 90 and 91 (quad 22, lane groups 2 and 3) hold no rows: zero
        if (beta + 2 >= uint32_t(mx::blocks) && beta < uint32_t(mx::blocks)) {
            const size_t zoff = off + 2 * 16 * 16;
#pragma unroll
            for (int p = 0; p < HP; ++p) {
                *reinterpret_cast<uint4 *>(hb + size_t(p) * mf::plane_bytes + zoff) = make_uint4(0, 0, 0, 0);
            }
        }
    }
}

template <int PX, bool F16H, class VX = bf16x8>
__global__ __launch_bounds__(kGuWaves * 64) __attribute__((amdgpu_waves_per_eu(2))) void gateup_kernel(GateUpArgs a) {
    __shared__ mf::u32x4 lds[2][Stager<PX, kGuWaves * 64>::lds_chunks];
    uint32_t tile, row_group;
    bool narrow;
    if (!tile_of_workgroup(a.plan.header, tile, row_group, narrow)) {
        return;
    }
    if (narrow) {
        gateup_tile<PX, kNarrowCols, F16H, VX>(a, tile, row_group, lds);
    } else {
        gateup_tile<PX, mf::col_tiles, F16H, VX>(a, tile, row_group, lds);
    }
}

// ---- plain GEMM (down projection, selected matmul) -----------------------------------------

struct MatmulArgs {
    const uint8_t *codes, *scales;
    const float *bias;  // [experts][rows] or null
    uint32_t rows, tiles_per_expert;
    const uint8_t *frags;  // [tile][tile_planes][plane_bytes], the GEMM reading the first P planes
    uint32_t tile_planes;
    Plan plan;
    float *out;          // SCATTER: [x_rows][rows] by token; else [slots][rows] by slot
    uint32_t out_rows;   // SCATTER: rows of out (tokens beyond are skipped)
};

// V: the operand type (bf16x8, or f16x8 for the hidden's two f16 planes); the B operand
// then holds its values times 2^SHIFT, so the accumulator starts at bias x 2^SHIFT and is
// scaled back at the store (powers of two: exact).
template <int P, bool SCATTER, int NC, class V, int SHIFT>
__device__ __attribute__((always_inline)) inline void matmul_tile(const MatmulArgs &a, uint32_t tile,
                                                                  uint32_t row_group,
                                                                  mf::u32x4 (*lds)[Stager<P, kMmWaves * 64>::lds_chunks]) {
    using SS = StageShape<P>;
    constexpr int kThreads = kMmWaves * 64;
    const uint32_t t = threadIdx.x, wave = t / 64, lane = t % 64;
    const uint32_t expert = a.plan.tile_expert[tile];
    const uint32_t row0 = row_group * kMmRows + wave * (kMmTiles * 16);
    const bool rows_ok = row0 < a.rows;  // waves past the last row only help stage
    const uint32_t row_base = rows_ok ? row0 : 0;
    const size_t tile0 = size_t(expert) * a.tiles_per_expert + row_base / 16;
    const uint8_t *frags = a.frags + size_t(tile) * a.tile_planes * mf::plane_bytes;

    AOperand<kMmTiles> wa;
    size_t ti[kMmTiles];
#pragma unroll
    for (int m = 0; m < kMmTiles; ++m) {
        ti[m] = tile0 + m;
    }
    wa.init(a.codes, a.scales, ti, lane);

    f32x4 acc[kMmTiles][NC];
    {
        const uint32_t g = lane / 16;
#pragma unroll
        for (int m = 0; m < kMmTiles; ++m) {
            f32x4 b = {0.f, 0.f, 0.f, 0.f};
            if (a.bias) {
                const float4 v =
                    *reinterpret_cast<const float4 *>(a.bias + size_t(expert) * a.rows + row_base + 16 * m + 4 * g);
                b = f32x4{v.x, v.y, v.z, v.w};
                if constexpr (SHIFT != 0) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        b[k] = __builtin_amdgcn_ldexpf(b[k], SHIFT);
                    }
                }
            }
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                acc[m][c] = b;
            }
        }
    }

    Stager<P, kThreads> st;
    st.load(frags, 0, t);
    uint4 qa[3][kMmTiles];
    wa.load(0, lane, qa[0]);
    wa.load(1, lane, qa[1]);
    st.store(lds[0], t);
    __syncthreads();
    if (SS::count > 1) {
        st.load(frags, 1, t);
    }

    auto stage_end = [&](int stage) __attribute__((always_inline)) {
        if (stage + 1 < SS::count) {
            st.store(lds[(stage + 1) % 2], t);
        }
        __syncthreads();
        if (stage + 2 < SS::count) {
            st.load(frags, stage + 2, t);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    auto compute_quad = [&](int i, const uint4(&q)[kMmTiles]) __attribute__((always_inline)) {
        float sc[kMmTiles];
#pragma unroll
        for (int m = 0; m < kMmTiles; ++m) {
            sc[m] = wa.scale(m);
        }
        wa.next_quad();
        auto decode = [&](int s, V(&w)[kMmTiles]) __attribute__((always_inline)) {
#pragma unroll
            for (int m = 0; m < kMmTiles; ++m) {
                const uint32_t word = s == 0 ? q[m].x : (s == 1 ? q[m].y : (s == 2 ? q[m].z : q[m].w));
                w[m] = mf::decode_as<V>(word, sc[m]);
            }
        };
        quad_mfma<P, kMmTiles, 4, NC, V>(lds[0], lds[1], i, lane, decode, stage_end, acc);
    };

    for (int i = 0; i < mf::quads; i += 3) {
        wa.load(min(i + 2, mf::quads - 1), lane, qa[2]);
        __builtin_amdgcn_sched_barrier(0);
        compute_quad(i, qa[0]);
        wa.load(min(i + 3, mf::quads - 1), lane, qa[0]);
        __builtin_amdgcn_sched_barrier(0);
        if (i + 1 < mf::quads) {
            compute_quad(i + 1, qa[1]);
            wa.load(min(i + 4, mf::quads - 1), lane, qa[1]);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (i + 2 < mf::quads) {
            compute_quad(i + 2, qa[2]);
        }
    }

    if (!rows_ok) {
        return;
    }
    const uint32_t cnt = a.plan.tile_count[tile], first = a.plan.tile_first[tile];
    const uint32_t g = lane / 16, n16 = lane % 16;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const uint32_t n = c * 16 + n16;
        if (n >= cnt) {
            continue;
        }
        size_t out_row;
        if (SCATTER) {
            const uint32_t token = a.plan.slot_token[first + n];
            if (token >= a.out_rows) {
                continue;
            }
            out_row = token;
        } else {
            out_row = first + n;
        }
        float *dst = a.out + out_row * a.rows + row0 + 4 * g;
#pragma unroll
        for (int m = 0; m < kMmTiles; ++m) {
            f32x4 v = acc[m][c];
            if constexpr (SHIFT != 0) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    v[k] = __builtin_amdgcn_ldexpf(v[k], -SHIFT);
                }
            }
            *reinterpret_cast<float4 *>(dst + 16 * m) = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
}

template <int P, bool SCATTER, class V = bf16x8, int SHIFT = 0>
__global__ __launch_bounds__(kMmWaves * 64) void matmul_kernel(MatmulArgs a) {
    __shared__ mf::u32x4 lds[2][Stager<P, kMmWaves * 64>::lds_chunks];
    uint32_t tile, row_group;
    bool narrow;
    if (!tile_of_workgroup(a.plan.header, tile, row_group, narrow)) {
        return;
    }
    if (narrow) {
        matmul_tile<P, SCATTER, kNarrowCols, V, SHIFT>(a, tile, row_group, lds);
    } else {
        matmul_tile<P, SCATTER, mf::col_tiles, V, SHIFT>(a, tile, row_group, lds);
    }
}

// ---- the scaled path: MXFP4 weights x MXFP8 activations on v_mfma_scale ------------------
//
// Activations (the gathered tokens, and the SwiGLU hidden between the two GEMMs) are
// quantized per 32-element block to MXFP8: E8M0 exponent X = the smallest with
// max|x| / 2^X <= 448 (mx8::block_exponent), elements E4M3 of x / 2^X rounded to
// nearest even.  One instruction then takes a whole quad (4 blocks) of 16 rows x 16
// tokens, with the weights' own bytes and scales as the A operand (no decode).  The
// products are those of the dequantized activations, but the instruction does not
// accumulate exactly in f32 (see mx8 in ttl_mfma.hpp): this path is the fast one,
// the bf16 one the exact one.

// The MXFP8 form of one block of 32 values: its exponent, or non-finite.
struct Mx8Block {
    int exponent;
    bool finite;
};

__device__ inline Mx8Block mx8_block(const float (&v)[32]) {
    float m = 0.0f;
    bool finite = true;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        finite = finite && isfinite(v[j]);
        m = fmaxf(m, fabsf(v[j]));
    }
    // a zero block takes scale 2^0; its codes are zero whatever the scale
    return {m > 0.0f ? mx8::block_exponent(m) : 0, finite};
}

__device__ inline uint32_t mx8_code(float v, const Mx8Block &b) {
    return b.finite ? mx8::e4m3(__builtin_amdgcn_ldexpf(v, -b.exponent)) : mx8::e4m3_nan;
}

// One workgroup per (quad, column tile, token tile); 16 threads per slot, 4 per
// 32-element block, each thread 8 consecutive elements (one 16-byte bf16 load, the
// slot's 4 blocks of the quad contiguous across its 16 threads).  The tile's metadata
// and the early exit are requested together, then the slot's token, then its row
// (unconditional requests at clamped addresses, masked after), so a thread waits for
// three dependent loads in all.  (One workgroup for the four column tiles in turn was
// slower: 10.2 against 8.5 us per launch.)  The block's largest magnitude takes two
// lane exchanges.  Element e of K-block g belongs to B lane group 2 (g & 1) +
// (e % 16) / 8, byte 16 (g >> 1) + 2 (e % 8) + e / 16, so the threads holding elements
// 8r..8r+7 and 8r+16..8r+23 (r = 0, 1) interleave their codes and the first writes 16
// contiguous bytes; the block's first thread writes its E8M0 byte, read by the MFMA
// from lane (n, g).  Slots past the tile's count and blocks 90/91 are zero; a token out
// of range is NaN.
template <bool BF16_IN>
__global__ __launch_bounds__(256) void gather_mx8_kernel(const void *__restrict__ x, uint32_t x_stride,
                                                          uint32_t x_rows, Plan plan) {
    const uint32_t tile = blockIdx.y;
    // (tile < the layout's tmax: its metadata words exist, stale past the plan's tiles)
    const uint32_t tiles = plan.header->tiles, count = plan.tile_count[tile], first = plan.tile_first[tile];
    if (tile >= tiles) {
        return;
    }
    const uint32_t quad = blockIdx.x / mf::col_tiles, ct = blockIdx.x % mf::col_tiles;
    const uint32_t t = threadIdx.x, n16 = t / 16, g = (t % 16) / 4, r = t % 4;
    const uint32_t n = ct * 16 + n16, block = 4 * quad + g;
    const bool block_ok = block < uint32_t(mx::blocks);
    const bool live = n < count && block_ok;
    const uint32_t token = plan.slot_token[first + min(n, count - 1)];
    const size_t base = size_t(token < x_rows ? token : 0u) * x_stride + size_t(block_ok ? block : 0u) * 32 + 8 * r;
    float v[8];
    if (BF16_IN) {
        const uint4 w = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(x) + base);
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[2 * k] = __uint_as_float(ww[k] << 16);
            v[2 * k + 1] = __uint_as_float(ww[k] & 0xffff0000u);
        }
    } else {
        const float4 *src = reinterpret_cast<const float4 *>(static_cast<const float *>(x) + base);
        const float4 w0 = src[0], w1 = src[1];
        const float ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            v[k] = ww[k];
        }
    }
    const bool nan_row = live && token >= x_rows;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        v[k] = nan_row ? __builtin_nanf("") : (live ? v[k] : 0.0f);
    }
    float m = 0.0f;
    int finite = 1;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        finite &= isfinite(v[k]) ? 1 : 0;
        m = fmaxf(m, fabsf(v[k]));
    }
    m = fmaxf(m, __shfl_xor(m, 1));
    m = fmaxf(m, __shfl_xor(m, 2));
    finite &= __shfl_xor(finite, 1);
    finite &= __shfl_xor(finite, 2);
    const Mx8Block blk{m > 0.0f ? mx8::block_exponent(m) : 0, finite != 0};
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        lo |= mx8_code(v[k], blk) << (8 * k);
        hi |= mx8_code(v[4 + k], blk) << (8 * k);
    }
    // the partner thread (r ^ 2) holds the elements 16 further on
    const uint32_t plo = uint32_t(__shfl_xor(int(lo), 2)), phi = uint32_t(__shfl_xor(int(hi), 2));
    uint8_t *tb = plan.xb + size_t(tile) * mf::plane_bytes;
    if (r < 2) {
        // bytes 2j and 2j + 1 = this thread's element j and the partner's
        const auto mix = [](uint32_t a, uint32_t b) __attribute__((always_inline)) {
            return (a & 0xffu) | ((b & 0xffu) << 8) | ((a & 0xff00u) << 8) | ((b & 0xff00u) << 16);
        };
        const uint4 out = make_uint4(mix(lo, plo), mix(lo >> 16, plo >> 16), mix(hi, phi), mix(hi >> 16, phi >> 16));
        const uint32_t dest = n16 + 16 * (2 * (g & 1) + r);
        *reinterpret_cast<uint4 *>(tb + ((size_t(quad) * mf::col_tiles + ct) * 64 + dest) * mx8::lane_bytes +
                                   16 * (g >> 1)) = out;
    }
    if (r == 0) {
        tb[mx8::tile_frag_bytes + (size_t(ct) * 64 + n16 + 16 * g) * mx8::scale_pad + quad] =
            uint8_t((blk.finite ? blk.exponent : 0) + 127);
    }
}

// B staging of the scaled kernels: kMx8StageQuads quads of all column tiles per LDS stage.
constexpr int kMx8StageQuads = 2;
constexpr size_t kMx8StageBytes = size_t(kMx8StageQuads) * mf::col_tiles * mx8::frag_bytes;  // 16 KiB

template <int THREADS>
struct Mx8Stager {
    static constexpr int pieces = int(kMx8StageBytes / 16);
    static constexpr int per = pieces / THREADS;
    static_assert(pieces % THREADS == 0, "whole pieces per thread");
    mf::u32x4 r[per];
    // pieces past the tile's last quad (the last stage's second half, and the stage after
    // the last that the main loop requests) re-read its last piece
    __device__ inline void load(const uint8_t *__restrict__ tile_frags, int stage, uint32_t t) {
#pragma unroll
        for (int k = 0; k < per; ++k) {
            const size_t off = min(size_t(stage) * kMx8StageBytes + (size_t(t) + size_t(k) * THREADS) * 16,
                                   mx8::tile_frag_bytes - 16);
            r[k] = *reinterpret_cast<const mf::u32x4 *>(tile_frags + off);
        }
    }
    // LDS holds each (quad, column tile) fragment as its 64 lanes' first 16 bytes, then
    // their last 16: a lane's two reads are then contiguous across the wave (the
    // fragment's own order, 32 bytes per lane, puts two lanes on the same banks)
    __device__ inline void store(mf::u32x4 *lds, uint32_t t) const {
#pragma unroll
        for (int k = 0; k < per; ++k) {
            const uint32_t piece = t + uint32_t(k) * THREADS, r16 = piece % 128;
            lds[piece - r16 + (r16 % 2) * 64 + r16 / 2] = r[k];
        }
    }
};

// One quad of the scaled main loop: B fragments of quad i from LDS (stage buffer
// i / 2 % 2), the A and B scale bytes of the quad, then M x NC instructions, tile by
// tile: as soon as tile m's instructions are issued, its registers take the codes of
// quad `next` (sched_barrier keeps each request at its place; left to the scheduler,
// the requests sank below the next quad's instructions and every wave waited for all
// of its loads, vmcnt(0), once per stage).  At the end of a stage (stage_end, a
// constant after unrolling) the next stage is published and the one after requested;
// past the last stage the request re-reads the plane's last piece (no condition
// around a load: the compiler would wait for it at once).
template <int M, int NC, int THREADS>
__device__ __attribute__((always_inline)) inline void mx8_quad(int i, uint4 (&q)[M], int next, AOperand<M> &wa,
                                                               uint32_t (&sb)[NC][6], Mx8Stager<THREADS> &st,
                                                               const uint8_t *tile_frags,
                                                               mf::u32x4 (*lds)[kMx8StageBytes / 16], uint32_t t,
                                                               uint32_t lane, mf::f32x4 (&acc)[M][NC], bool stage_end) {
    const int stage = i / kMx8StageQuads;
    const mf::u32x4 *buf = lds[stage % 2] + size_t(i % kMx8StageQuads) * mf::col_tiles * 64 * 2;
    mx8::i32x8 b[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const mf::u32x4 lo = buf[c * 128 + lane], hi = buf[c * 128 + 64 + lane];
        b[c] = mx8::i32x8{int32_t(lo[0]), int32_t(lo[1]), int32_t(lo[2]), int32_t(lo[3]),
                          int32_t(hi[0]), int32_t(hi[1]), int32_t(hi[2]), int32_t(hi[3])};
    }
    uint32_t sa[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        sa[m] = wa.scale_byte(m);
    }
    uint32_t scb[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        scb[c] = sb[c][0] & 0xffu;
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            acc[m][c] = mx8::mfma(q[m], b[c], sa[m], scb[c], acc[m][c]);
        }
        // tile m's codes are consumed: request quad `next` into the same registers
        __builtin_amdgcn_sched_barrier(0);
        q[m] = wa.load_one(next, lane, m);
        __builtin_amdgcn_sched_barrier(0);
    }
    wa.next_quad();
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
        for (int j = 0; j < 5; ++j) {
            sb[c][j] = (sb[c][j] >> 8) | (sb[c][j + 1] << 24);
        }
        sb[c][5] >>= 8;
    }
    if (stage_end) {
        st.store(lds[(stage + 1) % 2], t);
        __syncthreads();
        st.load(tile_frags, stage + 2, t);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// The scaled main loop of one wave: M 16-row A tiles (AOperand), NC column tiles, the
// B fragments staged in LDS by every wave of the workgroup.  acc[m][c] += A_m B_c for
// quads 0..22; two code buffers, each refilled tile by tile two quads ahead while the
// other quad is multiplied (a third buffer would cost the second wave per SIMD).
// Pairs of quads keep the buffer and stage-end positions static.
template <int M, int NC, int THREADS>
__device__ __attribute__((always_inline)) inline void mx8_main_loop(AOperand<M> &wa, const uint8_t *tile_frags,
                                                                    const uint8_t *tile_scales,
                                                                    mf::u32x4 (*lds)[kMx8StageBytes / 16], uint32_t t,
                                                                    uint32_t lane, mf::f32x4 (&acc)[M][NC]) {
    static_assert(kMx8StageQuads == 2, "a stage ends at every second quad");
    constexpr int full = mf::quads / 2 * 2;
    // the lane's B scale bytes per column tile (quads 0..22, shifted one byte per quad)
    uint32_t sb[NC][6];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const uint2 *rec = reinterpret_cast<const uint2 *>(tile_scales + (size_t(c) * 64 + lane) * mx8::scale_pad);
        const uint2 r0 = rec[0], r1 = rec[1], r2 = rec[2];
        sb[c][0] = r0.x;
        sb[c][1] = r0.y;
        sb[c][2] = r1.x;
        sb[c][3] = r1.y;
        sb[c][4] = r2.x;
        sb[c][5] = r2.y;
    }
    Mx8Stager<THREADS> st;
    st.load(tile_frags, 0, t);
    uint4 q[2][M];
    wa.load(0, lane, q[0]);
    wa.load(1, lane, q[1]);
    st.store(lds[0], t);
    __syncthreads();
    st.load(tile_frags, 1, t);
    for (int i = 0; i < full; i += 2) {
        mx8_quad<M, NC, THREADS>(i, q[0], i + 2, wa, sb, st, tile_frags, lds, t, lane, acc, false);
        mx8_quad<M, NC, THREADS>(i + 1, q[1], min(i + 3, mf::quads - 1), wa, sb, st, tile_frags, lds, t, lane, acc,
                                 true);
    }
    static_assert(mf::quads - full == 1, "one quad after the pairs");
    mx8_quad<M, NC, THREADS>(full, q[0], full, wa, sb, st, tile_frags, lds, t, lane, acc, false);
}

// Gate/up on the scaled path, the workgroup layout of gateup_kernel (4 waves x 32 rows:
// gate and up of two 16-row tiles per wave).  The SwiGLU hidden of a wave's 32 rows is
// one 32-element K-block beta of the down GEMM for each token: lanes (n, 0..3) hold its
// rows 4g..4g+3 and 16+4g..16+4g+3, so the block's maximum takes two lane exchanges,
// and each lane writes 8 contiguous fp8 bytes of the down GEMM's B fragment.
template <int NC>
__device__ __attribute__((always_inline)) inline void mx8_gateup_tile(const GateUpArgs &a, uint32_t tile,
                                                                      uint32_t row_group,
                                                                      mf::u32x4 (*lds)[kMx8StageBytes / 16]) {
    constexpr int kThreads = kGuWaves * 64;
    const uint32_t t = threadIdx.x, wave = t / 64, lane = t % 64;
    const uint32_t expert = a.plan.tile_expert[tile];
    const uint32_t row0 = row_group * kGuRows + wave * 32;
    const bool rows_ok = row0 < a.rows;
    const uint32_t row_base = rows_ok ? row0 : row_group * kGuRows;
    const size_t tile0 = size_t(expert) * a.tiles_per_expert + row_base / 16;
    const uint8_t *tb = a.plan.xb + size_t(tile) * mf::plane_bytes;

    // A tiles: gate rows +0, +16, up rows +0, +16 (AOperand over both tensors)
    AOperand<4> wa;
    {
        AOperand<2> ga, ua;
        const size_t ti[2] = {tile0, tile0 + 1};
        ga.init(a.gate_codes, a.gate_scales, ti, lane);
        ua.init(a.up_codes, a.up_scales, ti, lane);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            wa.codes[k] = ga.codes[k];
            wa.codes[2 + k] = ua.codes[k];
#pragma unroll
            for (int j = 0; j < 6; ++j) {
                wa.sw[k][j] = ga.sw[k][j];
                wa.sw[2 + k][j] = ua.sw[k][j];
            }
        }
    }
    mf::f32x4 acc[4][NC];
    {
        const uint32_t g = lane / 16;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const float *bias = m < 2 ? a.gate_bias : a.up_bias;
            mf::f32x4 b = {0.f, 0.f, 0.f, 0.f};
            if (bias) {
                const float4 v = *reinterpret_cast<const float4 *>(bias + size_t(expert) * a.rows + row_base +
                                                                   16 * (m % 2) + 4 * g);
                b = mf::f32x4{v.x, v.y, v.z, v.w};
            }
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                acc[m][c] = b;
            }
        }
    }
    mx8_main_loop<4, NC, kThreads>(wa, tb, tb + mx8::tile_frag_bytes, lds, t, lane, acc);
    if (!rows_ok) {
        return;
    }
    // the hidden block beta = this wave's 32 rows: K-block g = beta % 4 of quad beta / 4
    const uint32_t beta = row0 / 32, quad = beta / 4, gk = beta % 4;
    const uint32_t gs = lane / 16, n16 = lane % 16;
    uint8_t *hb = a.plan.hb + size_t(tile) * mf::plane_bytes;
    // bytes 16 (g>>1) + 8 (gs%2) .. +7 of B lane (n, 2 (g&1) + gs/2)
    const auto dest = [&](uint32_t g, uint32_t c) __attribute__((always_inline)) {
        return hb + ((size_t(quad) * mf::col_tiles + c) * 64 + n16 + 16 * (2 * (g & 1) + gs / 2)) * mx8::lane_bytes +
               16 * (g >> 1) + 8 * (gs % 2);
    };
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        float h[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            h[2 * i] = moe_math::clamped_swiglu_fast(acc[0][c][i], acc[2][c][i]);      // element 4 gs + i
            h[2 * i + 1] = moe_math::clamped_swiglu_fast(acc[1][c][i], acc[3][c][i]);  // element 16 + 4 gs + i
        }
        float m = 0.0f;
        bool finite = true;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            finite = finite && isfinite(h[j]);
            m = fmaxf(m, fabsf(h[j]));
        }
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
        int fin = finite ? 1 : 0;
        fin &= __shfl_xor(fin, 16);
        fin &= __shfl_xor(fin, 32);
        const Mx8Block blk{m > 0.0f ? mx8::block_exponent(m) : 0, fin != 0};
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            lo |= mx8_code(h[j], blk) << (8 * j);
            hi |= mx8_code(h[4 + j], blk) << (8 * j);
        }
        *reinterpret_cast<uint2 *>(dest(gk, c)) = make_uint2(lo, hi);
        if (gs == 0) {
            hb[mx8::tile_frag_bytes + (size_t(c) * 64 + n16 + 16 * gk) * mx8::scale_pad + quad] =
                uint8_t((blk.finite ? blk.exponent : 0) + 127);
        }
        // blocks 90 and 91 (K-blocks 2 and 3 of quad 22) hold no rows: zero, scale 2^0
        if (beta + 2 >= uint32_t(mx::blocks) && beta < uint32_t(mx::blocks)) {
            *reinterpret_cast<uint2 *>(dest(gk + 2, c)) = make_uint2(0u, 0u);
            if (gs == 0) {
                hb[mx8::tile_frag_bytes + (size_t(c) * 64 + n16 + 16 * (gk + 2)) * mx8::scale_pad + quad] = 127;
            }
        }
    }
}

__global__ __launch_bounds__(kGuWaves * 64) void mx8_gateup_kernel(GateUpArgs a) {
    __shared__ mf::u32x4 lds[2][kMx8StageBytes / 16];
    uint32_t tile, row_group;
    bool narrow;
    if (!tile_of_workgroup(a.plan.header, tile, row_group, narrow)) {
        return;
    }
    if (narrow) {
        mx8_gateup_tile<kNarrowCols>(a, tile, row_group, lds);
    } else {
        mx8_gateup_tile<mf::col_tiles>(a, tile, row_group, lds);
    }
}

// Down projection and the selected-token matmul on the scaled path: matmul_kernel's
// workgroup layout (4 waves x 48 rows) and epilogue; B from frags (gather or gate/up).
template <bool SCATTER, int NC>
__device__ __attribute__((always_inline)) inline void mx8_matmul_tile(const MatmulArgs &a, uint32_t tile,
                                                                      uint32_t row_group,
                                                                      mf::u32x4 (*lds)[kMx8StageBytes / 16]) {
    constexpr int kThreads = kMmWaves * 64;
    const uint32_t t = threadIdx.x, wave = t / 64, lane = t % 64;
    const uint32_t expert = a.plan.tile_expert[tile];
    const uint32_t row0 = row_group * kMmRows + wave * (kMmTiles * 16);
    const bool rows_ok = row0 < a.rows;
    const uint32_t row_base = rows_ok ? row0 : 0;
    const size_t tile0 = size_t(expert) * a.tiles_per_expert + row_base / 16;
    const uint8_t *tb = a.frags + size_t(tile) * mf::plane_bytes;
    AOperand<kMmTiles> wa;
    size_t ti[kMmTiles];
#pragma unroll
    for (int m = 0; m < kMmTiles; ++m) {
        ti[m] = tile0 + m;
    }
    wa.init(a.codes, a.scales, ti, lane);
    mf::f32x4 acc[kMmTiles][NC];
    {
        const uint32_t g = lane / 16;
#pragma unroll
        for (int m = 0; m < kMmTiles; ++m) {
            mf::f32x4 b = {0.f, 0.f, 0.f, 0.f};
            if (a.bias) {
                const float4 v =
                    *reinterpret_cast<const float4 *>(a.bias + size_t(expert) * a.rows + row_base + 16 * m + 4 * g);
                b = mf::f32x4{v.x, v.y, v.z, v.w};
            }
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                acc[m][c] = b;
            }
        }
    }
    mx8_main_loop<kMmTiles, NC, kThreads>(wa, tb, tb + mx8::tile_frag_bytes, lds, t, lane, acc);
    if (!rows_ok) {
        return;
    }
    const uint32_t cnt = a.plan.tile_count[tile], first = a.plan.tile_first[tile];
    const uint32_t g = lane / 16, n16 = lane % 16;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const uint32_t n = c * 16 + n16;
        if (n >= cnt) {
            continue;
        }
        size_t out_row;
        if (SCATTER) {
            const uint32_t token = a.plan.slot_token[first + n];
            if (token >= a.out_rows) {
                continue;
            }
            out_row = token;
        } else {
            out_row = first + n;
        }
        float *dst = a.out + out_row * a.rows + row0 + 4 * g;
#pragma unroll
        for (int m = 0; m < kMmTiles; ++m) {
            *reinterpret_cast<float4 *>(dst + 16 * m) = make_float4(acc[m][c][0], acc[m][c][1], acc[m][c][2],
                                                                    acc[m][c][3]);
        }
    }
}

template <bool SCATTER>
__global__ __launch_bounds__(kMmWaves * 64) void mx8_matmul_kernel(MatmulArgs a) {
    __shared__ mf::u32x4 lds[2][kMx8StageBytes / 16];
    uint32_t tile, row_group;
    bool narrow;
    if (!tile_of_workgroup(a.plan.header, tile, row_group, narrow)) {
        return;
    }
    if (narrow) {
        mx8_matmul_tile<SCATTER, kNarrowCols>(a, tile, row_group, lds);
    } else {
        mx8_matmul_tile<SCATTER, mf::col_tiles>(a, tile, row_group, lds);
    }
}

// The values the scaled path multiplies: each row's 32-element blocks quantized to
// MXFP8 and widened back to f32 (one thread per block).
template <bool BF16_IN>
__global__ __launch_bounds__(256) void mx8_dequantize_kernel(const void *__restrict__ x, uint32_t rows,
                                                             float *__restrict__ out) {
    const size_t gid = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= size_t(rows) * mx::blocks) {
        return;
    }
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        v[j] = BF16_IN ? __uint_as_float(uint32_t(static_cast<const uint16_t *>(x)[gid * 32 + j]) << 16)
                       : static_cast<const float *>(x)[gid * 32 + j];
    }
    const Mx8Block b = mx8_block(v);
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const uint32_t code = mx8_code(v[j], b);
        out[gid * 32 + j] = b.finite ? __builtin_amdgcn_ldexpf(mx8::e4m3_value(code), b.exponent) : __builtin_nanf("");
    }
}

// ---- the intermediates, read back for inspection -----------------------------------------

// One workgroup per (token, rank) pair p: the pair's SwiGLU hidden as the down GEMM
// reads it (the MXFP8 codes times their E8M0 scale on the scaled path; the sum of the
// three bf16 planes, or of the two f16 planes scaled back by 2^-kHiddenF16Shift, on the
// exact one) and its down row (bias included, before the routing
// weight), from the workspace a full prefill left.  A pair without a slot (invalid
// expert index) gets NaN rows.  The slot's tile is found by a scan of the plan's tiles.
template <bool SCALED, bool F16H>
__global__ __launch_bounds__(256) void prefill_intermediates_kernel(Plan plan, uint32_t rows,
                                                                    float *__restrict__ hidden_out,
                                                                    float *__restrict__ down_out,
                                                                    uint8_t *__restrict__ scales_out) {
    const uint32_t p = blockIdx.x, t = threadIdx.x;
    const int32_t slot = plan.pair_slot[p];
    float *h = hidden_out + size_t(p) * mx::cols;
    float *d = down_out + size_t(p) * rows;
    if (slot < 0) {
        for (uint32_t k = t; k < uint32_t(mx::cols); k += blockDim.x) {
            h[k] = __builtin_nanf("");
        }
        for (uint32_t k = t; k < rows; k += blockDim.x) {
            d[k] = __builtin_nanf("");
        }
        return;
    }
    const uint32_t s = uint32_t(slot), tiles = plan.header->tiles;
    uint32_t tile = 0;
    for (uint32_t i = 0; i < tiles; ++i) {
        const uint32_t f = plan.tile_first[i];
        tile = (s >= f && s < f + plan.tile_count[i]) ? i : tile;
    }
    const uint32_t n = s - plan.tile_first[tile], c = n / 16, n16 = n % 16;
    for (uint32_t k = t; k < uint32_t(mx::cols); k += blockDim.x) {
        const uint32_t beta = k / 32, e = k % 32, quad = beta / 4, g = beta % 4;
        float v;
        if (SCALED) {
            const uint8_t *hb = plan.hb + size_t(tile) * mf::plane_bytes;
            const uint32_t code =
                hb[((size_t(quad) * mf::col_tiles + c) * 64 + n16 + 16 * mx8::b_group(g, e)) * mx8::lane_bytes +
                   mx8::b_byte(g, e)];
            const uint32_t sc = hb[mx8::tile_frag_bytes + (size_t(c) * 64 + n16 + 16 * g) * mx8::scale_pad + quad];
            v = (code & 0x7fu) == mx8::e4m3_nan ? __builtin_nanf("")
                                                : __builtin_amdgcn_ldexpf(mx8::e4m3_value(code), int(sc) - 127);
            if (e == 0 && scales_out) {
                scales_out[size_t(p) * mx::blocks + beta] = uint8_t(sc);
            }
        } else {
            // element e of block beta: K step 4 quad + (e % 16) / 4, lane (beta % 4, n16),
            // value 2 (e % 4) + e / 16 of the lane's 8
            const uint8_t *hb = plan.hb + size_t(tile) * kHiddenPlanes * mf::plane_bytes;
            const size_t off = ((size_t(quad) * 4 + (e % 16) / 4) * mf::col_tiles + c) * mf::frag_bytes +
                               (g * 16 + n16) * 16 + 2 * (2 * (e % 4) + e / 16);
            auto half = [&](int pl) __attribute__((always_inline)) {
                return *reinterpret_cast<const uint16_t *>(hb + size_t(pl) * mf::plane_bytes + off);
            };
            if (F16H) {
                // the two f16 planes of h x 2^kHiddenF16Shift: their sum is exact in f32
                v = __builtin_amdgcn_ldexpf(float(__builtin_bit_cast(_Float16, half(0))) +
                                                float(__builtin_bit_cast(_Float16, half(1))),
                                            -mf::kHiddenF16Shift);
            } else {
                v = 0.0f;
#pragma unroll
                for (int pl = 0; pl < kHiddenPlanes; ++pl) {
                    v += __uint_as_float(uint32_t(half(pl)) << 16);
                }
            }
        }
        h[k] = v;
    }
    for (uint32_t k = t; k < rows; k += blockDim.x) {
        d[k] = plan.down[size_t(s) * rows + k];
    }
}

// ---- combine ----------------------------------------------------------------------------

// out[p][i] = sum over token p's slots in slot order (= expert order) of
// weight * down[slot][i]: products rounded, then added to a running sum from +0
// (model.cpp:380, 450-459).  A pair with an invalid expert index makes the token NaN.
// USED is the pairs per token (the sort is a fixed network over USED registers).
template <int USED>
__global__ __launch_bounds__(256) void combine_kernel(Plan plan, uint32_t count, uint32_t rows,
                                                      const float *__restrict__ residual, float *__restrict__ out) {
#pragma clang fp contract(off)
    const uint32_t quads_per_row = rows / 4;
    const size_t gid = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= size_t(count) * quads_per_row) {
        return;
    }
    const uint32_t p = uint32_t(gid / quads_per_row), q = uint32_t(gid % quads_per_row);
    int32_t slots[USED];
    bool bad = false;
#pragma unroll
    for (int r = 0; r < USED; ++r) {
        slots[r] = plan.pair_slot[size_t(p) * USED + r];
        bad |= slots[r] < 0;
    }
    // ascending slot order: odd-even transposition sort over the registers
#pragma unroll
    for (int pass = 0; pass < USED; ++pass) {
#pragma unroll
        for (int i = pass % 2; i + 1 < USED; i += 2) {
            const int32_t lo = min(slots[i], slots[i + 1]), hi = max(slots[i], slots[i + 1]);
            slots[i] = lo;
            slots[i + 1] = hi;
        }
    }
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (bad) {
        const float nan = __builtin_nanf("");
        acc = make_float4(nan, nan, nan, nan);
    } else {
#pragma unroll
        for (int r = 0; r < USED; ++r) {
            const uint32_t s = uint32_t(slots[r]);
            const float w = plan.slot_weight[s];
            const float4 d = reinterpret_cast<const float4 *>(plan.down + size_t(s) * rows)[q];
            acc.x = acc.x + w * d.x;
            acc.y = acc.y + w * d.y;
            acc.z = acc.z + w * d.z;
            acc.w = acc.w + w * d.w;
        }
    }
    if (residual) {
        // model.cpp:545-551: x = residual + moe
        const float4 r = reinterpret_cast<const float4 *>(residual + size_t(p) * rows)[q];
        acc = make_float4(r.x + acc.x, r.y + acc.y, r.z + acc.z, r.w + acc.w);
    }
    reinterpret_cast<float4 *>(out + size_t(p) * rows)[q] = acc;
}

template <int USED>
void launch_combine(const Plan &plan, uint32_t count, uint32_t rows, const float *residual, float *out,
                    hipStream_t stream) {
    const size_t threads = size_t(count) * (rows / 4);
    combine_kernel<USED><<<unsigned((threads + 255) / 256), 256, 0, stream>>>(plan, count, rows, residual, out);
}

// Dispatches the combine on the number of pairs per token (1..16).
template <int U = 1>
void combine_for(uint32_t used, const Plan &plan, uint32_t count, uint32_t rows, const float *residual, float *out,
                 hipStream_t stream) {
    if constexpr (U <= int(kMaxUsed)) {
        if (used == uint32_t(U)) {
            launch_combine<U>(plan, count, rows, residual, out, stream);
        } else {
            combine_for<U + 1>(used, plan, count, rows, residual, out, stream);
        }
    }
}

// The MFMA kernels take weights as bf16 = E2M1 x 2^(e-127), exact for E8M0 1..254
// (and for zero codes at E8M0 0) only.  expert < 0: every expert of the tensor.
// The exact path's hidden between gate/up and down: two f16 planes (down decoded to f16,
// two thirds of the three-plane MFMAs) when every down expert's scales keep its f16
// decode exact, else three bf16 planes.
bool hidden_f16(const ttl_moe_layer &L) {
    return L.down->f16_exact();
}

int check_bf16_scales(const ttl_mxfp4 *w, int64_t expert, const char *who) {
    const bool edge = expert < 0 ? w->edge_scales() : w->edge_experts[size_t(expert)] != 0;
    TTL_REQUIRE(!edge, TTL_ERR_SHAPE,
                "%s: the expert tensor has blocks with E8M0 scale 0 or 255, which the bf16 MFMA decode cannot "
                "represent exactly; use the matvec entry points for it",
                who);
    return TTL_OK;
}

int check_mxfp4(const ttl_mxfp4 *w, const char *who) {
    TTL_REQUIRE(w && w->codes && w->scales, TTL_ERR_INVALID, "%s: null tensor", who);
    TTL_REQUIRE(w->cols == uint32_t(mx::cols), TTL_ERR_SHAPE, "%s: cols must be %d", who, mx::cols);
    return TTL_OK;
}

}  // namespace

namespace ttl {

int launch_row_shifts(hipStream_t stream, const float *x, uint32_t stride, uint32_t rows, uint32_t cols,
                      int32_t *shift) {
    TTL_REQUIRE(cols > 0 && cols <= kShiftMaxCols && cols % 4 == 0 && stride % 4 == 0 &&
                    (reinterpret_cast<uintptr_t>(x) & 15) == 0,
                TTL_ERR_SHAPE, "row shifts: rows of %u values, %u apart", cols, stride);
    if (rows == 0) {
        return TTL_OK;
    }
    row_shift_kernel<<<ttl::blocks_for(rows, kShiftRowsPerBlock), kShiftRowsPerBlock * 64, 0, stream>>>(
        x, stride, rows, cols, shift);
    TTL_LAUNCHED("row_shift_kernel");
    return TTL_OK;
}

}  // namespace ttl

extern "C" {

size_t ttl_matmul_mxfp4_selected_workspace_bytes(uint32_t count) {
    return make_layout(count, 1, 3, false, 0).total;
}

int ttl_matmul_mxfp4_selected(ttl_ctx *ctx, const ttl_mxfp4 *w, const float *bias_dev, const float *x_dev,
                              uint32_t x_stride, uint32_t x_rows, const int32_t *tokens_dev, uint32_t count,
                              float *out_dev, uint32_t expert, void *workspace_dev, size_t workspace_bytes) {
    TTL_REQUIRE(ctx && x_dev && tokens_dev && out_dev && workspace_dev, TTL_ERR_INVALID,
                "ttl_matmul_mxfp4_selected: null argument");
    int rc = check_mxfp4(w, "ttl_matmul_mxfp4_selected");
    if (rc != TTL_OK) {
        return rc;
    }
    TTL_REQUIRE(w->rows % kMmRows == 0, TTL_ERR_SHAPE, "ttl_matmul_mxfp4_selected: rows must be a multiple of %d",
                kMmRows);
    TTL_REQUIRE(expert < w->experts, TTL_ERR_INVALID, "ttl_matmul_mxfp4_selected: expert %u out of range", expert);
    rc = check_bf16_scales(w, expert, "ttl_matmul_mxfp4_selected");
    if (rc != TTL_OK) {
        return rc;
    }
    TTL_REQUIRE(x_stride >= uint32_t(mx::cols) && x_stride % 4 == 0, TTL_ERR_SHAPE,
                "ttl_matmul_mxfp4_selected: x_stride must be >= %d and a multiple of 4", mx::cols);
    TTL_REQUIRE((reinterpret_cast<uintptr_t>(x_dev) & 15) == 0 && (reinterpret_cast<uintptr_t>(out_dev) & 15) == 0,
                TTL_ERR_INVALID, "ttl_matmul_mxfp4_selected: x and out must be 16-byte aligned");
    TTL_REQUIRE(count <= kMaxEntries, TTL_ERR_SHAPE, "ttl_matmul_mxfp4_selected: count above %u", kMaxEntries);
    TTL_REQUIRE((reinterpret_cast<uintptr_t>(workspace_dev) & 255) == 0, TTL_ERR_INVALID,
                "ttl_matmul_mxfp4_selected: workspace must be 256-byte aligned");
    if (count == 0) {
        return TTL_OK;
    }
    const Layout L = make_layout(count, 1, 3, false, 0);
    TTL_REQUIRE(workspace_bytes >= L.total, TTL_ERR_SHAPE,
                "ttl_matmul_mxfp4_selected: workspace of %zu bytes, %zu needed", workspace_bytes, L.total);
    const Plan plan = plan_at(workspace_dev, L);
    const uint32_t tiles = (count + mf::tile_slots - 1) / mf::tile_slots;
    plan_selected_kernel<<<ttl::blocks_for(count > tiles ? count : tiles, 256), 256, 0, ctx->stream>>>(
        tokens_dev, count, expert, plan);
    TTL_LAUNCHED("plan_selected_kernel");
    gather_kernel<false, 3><<<dim3(mf::quads, tiles), mf::col_tiles * 64, 0, ctx->stream>>>(x_dev, x_stride, x_rows, plan);
    TTL_LAUNCHED("gather_kernel");
    MatmulArgs m;
    m.codes = w->codes;
    m.scales = w->scales;
    m.bias = bias_dev;
    m.rows = w->rows;
    m.tiles_per_expert = w->tiles;
    m.frags = plan.xb;
    m.tile_planes = 3;
    m.plan = plan;
    m.out = out_dev;
    m.out_rows = x_rows;
    matmul_kernel<3, true><<<dim3(w->rows / kMmRows, tiles), kMmWaves * 64, 0, ctx->stream>>>(m);
    TTL_LAUNCHED("matmul_kernel");
    return TTL_OK;
}

size_t ttl_matmul_mxfp4_selected_mxfp8_workspace_bytes(uint32_t count) {
    return make_layout(count, 1, 1, false, 0).total;
}

int ttl_matmul_mxfp4_selected_mxfp8(ttl_ctx *ctx, const ttl_mxfp4 *w, const float *bias_dev, const float *x_dev,
                                    uint32_t x_stride, uint32_t x_rows, const int32_t *tokens_dev, uint32_t count,
                                    float *out_dev, uint32_t expert, void *workspace_dev, size_t workspace_bytes) {
    const char *who = "ttl_matmul_mxfp4_selected_mxfp8";
    TTL_REQUIRE(ctx && x_dev && tokens_dev && out_dev && workspace_dev, TTL_ERR_INVALID, "%s: null argument", who);
    int rc = check_mxfp4(w, who);
    if (rc != TTL_OK) {
        return rc;
    }
    TTL_REQUIRE(w->rows % kMmRows == 0, TTL_ERR_SHAPE, "%s: rows must be a multiple of %d", who, kMmRows);
    TTL_REQUIRE(expert < w->experts, TTL_ERR_INVALID, "%s: expert %u out of range", who, expert);
    rc = check_bf16_scales(w, expert, who);
    if (rc != TTL_OK) {
        return rc;
    }
    TTL_REQUIRE(x_stride >= uint32_t(mx::cols) && x_stride % 4 == 0, TTL_ERR_SHAPE,
                "%s: x_stride must be >= %d and a multiple of 4", who, mx::cols);
    TTL_REQUIRE((reinterpret_cast<uintptr_t>(x_dev) & 15) == 0 && (reinterpret_cast<uintptr_t>(out_dev) & 15) == 0,
                TTL_ERR_INVALID, "%s: x and out must be 16-byte aligned", who);
    TTL_REQUIRE(count <= kMaxEntries, TTL_ERR_SHAPE, "%s: count above %u", who, kMaxEntries);
    TTL_REQUIRE((reinterpret_cast<uintptr_t>(workspace_dev) & 255) == 0, TTL_ERR_INVALID,
                "%s: workspace must be 256-byte aligned", who);
    if (count == 0) {
        return TTL_OK;
    }
    const Layout L = make_layout(count, 1, 1, false, 0);
    TTL_REQUIRE(workspace_bytes >= L.total, TTL_ERR_SHAPE, "%s: workspace of %zu bytes, %zu needed", who,
                workspace_bytes, L.total);
    const Plan plan = plan_at(workspace_dev, L);
    const uint32_t tiles = (count + mf::tile_slots - 1) / mf::tile_slots;
    plan_selected_kernel<<<ttl::blocks_for(count > tiles ? count : tiles, 256), 256, 0, ctx->stream>>>(
        tokens_dev, count, expert, plan);
    TTL_LAUNCHED("plan_selected_kernel");
    gather_mx8_kernel<false><<<dim3(mf::quads * mf::col_tiles, tiles), 256, 0, ctx->stream>>>(x_dev, x_stride,
                                                                                                  x_rows, plan);
    TTL_LAUNCHED("gather_mx8_kernel");
    MatmulArgs m;
    m.codes = w->codes;
    m.scales = w->scales;
    m.bias = bias_dev;
    m.rows = w->rows;
    m.tiles_per_expert = w->tiles;
    m.frags = plan.xb;
    m.tile_planes = 1;
    m.plan = plan;
    m.out = out_dev;
    m.out_rows = x_rows;
    mx8_matmul_kernel<true><<<dim3(w->rows / kMmRows, tiles), kMmWaves * 64, 0, ctx->stream>>>(m);
    TTL_LAUNCHED("mx8_matmul_kernel");
    return TTL_OK;
}

int ttl_mxfp8_dequantize(ttl_ctx *ctx, const void *x_dev, int x_dtype, uint32_t rows, float *out_dev) {
    TTL_REQUIRE(ctx && x_dev && out_dev, TTL_ERR_INVALID, "ttl_mxfp8_dequantize: null argument");
    TTL_REQUIRE(x_dtype == TTL_DTYPE_F32 || x_dtype == TTL_DTYPE_BF16, TTL_ERR_INVALID,
                "ttl_mxfp8_dequantize: x_dtype must be TTL_DTYPE_F32 or TTL_DTYPE_BF16");
    const size_t blocks = size_t(rows) * mx::blocks;
    if (blocks == 0) {
        return TTL_OK;
    }
    if (x_dtype == TTL_DTYPE_BF16) {
        mx8_dequantize_kernel<true><<<unsigned((blocks + 255) / 256), 256, 0, ctx->stream>>>(x_dev, rows, out_dev);
    } else {
        mx8_dequantize_kernel<false><<<unsigned((blocks + 255) / 256), 256, 0, ctx->stream>>>(x_dev, rows, out_dev);
    }
    TTL_LAUNCHED("mx8_dequantize_kernel");
    return TTL_OK;
}

size_t ttl_moe_prefill_workspace_bytes(uint32_t count, uint32_t experts, uint32_t used, int x_dtype) {
    const bool f32 = x_dtype == TTL_DTYPE_F32;
    const int planes = f32 ? 3 : 1;  // bf16, or the MXFP8 fragments (one plane's room)
    return make_layout(count * used, experts, planes, true, uint32_t(mx::cols), f32 ? count : 0).total;
}

}  // extern "C"

namespace {

// ttl_moe_prefill_stages with, for f32 tokens, their f16-plane shifts given (x_shift_dev,
// int32 [count], as ttl::launch_row_shifts computes them; else computed here) and the
// combine's residual add (residual_dev f32 [count][hidden], or null).
int moe_prefill_run(ttl_ctx *ctx, const ttl_moe_layer *layer, const void *x_dev, int x_dtype, uint32_t count,
                    const int32_t *indices_dev, const float *weights_dev, float *out_dev, void *workspace_dev,
                    size_t workspace_bytes, uint32_t stages, const int32_t *x_shift_dev, const float *residual_dev) {
    TTL_REQUIRE(ctx && layer && x_dev && indices_dev && weights_dev && out_dev && workspace_dev, TTL_ERR_INVALID,
                "ttl_moe_prefill_experts: null argument");
    TTL_REQUIRE((stages & ~uint32_t(TTL_PREFILL_ALL)) == 0, TTL_ERR_INVALID,
                "ttl_moe_prefill_stages: unknown stage bits 0x%x", stages);
    const ttl_moe_layer &L = *layer;
    TTL_REQUIRE(L.gate && L.up && L.down, TTL_ERR_INVALID, "ttl_moe_prefill_experts: null expert tensor");
    TTL_REQUIRE(x_dtype == TTL_DTYPE_F32 || x_dtype == TTL_DTYPE_BF16 || x_dtype == TTL_DTYPE_F32_AS_MXFP8 ||
                    x_dtype == TTL_DTYPE_BF16_AS_MXFP8,
                TTL_ERR_INVALID, "ttl_moe_prefill_experts: unknown x_dtype %d", x_dtype);
    TTL_REQUIRE(L.hidden == uint32_t(mx::cols) && L.expert_hidden == uint32_t(mx::cols), TTL_ERR_SHAPE,
                "ttl_moe_prefill_experts: hidden and expert_hidden must be %d", mx::cols);
    TTL_REQUIRE(L.gate->rows == L.expert_hidden && L.up->rows == L.expert_hidden && L.down->rows == L.hidden &&
                    L.gate->cols == L.hidden && L.up->cols == L.hidden && L.down->cols == L.expert_hidden,
                TTL_ERR_SHAPE, "ttl_moe_prefill_experts: expert tensor shapes do not match the layer");
    TTL_REQUIRE(L.gate->experts == L.experts && L.up->experts == L.experts && L.down->experts == L.experts,
                TTL_ERR_SHAPE, "ttl_moe_prefill_experts: expert tensors must hold %u experts", L.experts);
    for (const ttl_mxfp4 *t : {L.gate, L.up, L.down}) {
        const int rc = check_bf16_scales(t, -1, "ttl_moe_prefill_experts");
        if (rc != TTL_OK) {
            return rc;
        }
    }
    TTL_REQUIRE(L.experts >= 1 && L.experts <= kMaxExperts, TTL_ERR_SHAPE,
                "ttl_moe_prefill_experts: experts must be 1..%u", kMaxExperts);
    TTL_REQUIRE(L.used >= 1 && L.used <= kMaxUsed, TTL_ERR_SHAPE, "ttl_moe_prefill_experts: used must be 1..%u",
                kMaxUsed);
    TTL_REQUIRE(uint64_t(count) * L.used <= kMaxEntries, TTL_ERR_SHAPE,
                "ttl_moe_prefill_experts: count * used above %u", kMaxEntries);
    TTL_REQUIRE((reinterpret_cast<uintptr_t>(x_dev) & 15) == 0 && (reinterpret_cast<uintptr_t>(out_dev) & 15) == 0,
                TTL_ERR_INVALID, "ttl_moe_prefill_experts: x and out must be 16-byte aligned");
    TTL_REQUIRE((reinterpret_cast<uintptr_t>(workspace_dev) & 255) == 0, TTL_ERR_INVALID,
                "ttl_moe_prefill_experts: workspace must be 256-byte aligned");
    if (count == 0) {
        return TTL_OK;
    }
    const uint32_t pairs = count * L.used;
    const bool scaled = x_dtype == TTL_DTYPE_F32_AS_MXFP8 || x_dtype == TTL_DTYPE_BF16_AS_MXFP8;
    const bool bf16 = x_dtype == TTL_DTYPE_BF16 || x_dtype == TTL_DTYPE_BF16_AS_MXFP8;
    const bool f16h = !scaled && hidden_f16(L);
    // f32 tokens as two f16 planes of x 2^k (k per token) when the gate and up weights'
    // scales keep their f16 decode exact, else three exact bf16 planes
    const bool f32 = x_dtype == TTL_DTYPE_F32;
    const bool f16x = f32 && L.gate->f16_exact() && L.up->f16_exact();
    const Layout lay = make_layout(pairs, L.experts, (bf16 || scaled) ? 1 : 3, true, L.hidden, f32 ? count : 0);
    TTL_REQUIRE(workspace_bytes >= lay.total, TTL_ERR_SHAPE,
                "ttl_moe_prefill_experts: workspace of %zu bytes, %zu needed for this count and x_dtype",
                workspace_bytes, lay.total);
    const Plan plan = plan_at(workspace_dev, lay);

    if (stages & TTL_PREFILL_PLAN) {
        plan_kernel<<<1, kPlanThreads, 0, ctx->stream>>>(indices_dev, weights_dev, pairs, L.used, L.experts, plan);
        TTL_LAUNCHED("plan_kernel");
    }
    if ((stages & TTL_PREFILL_GATHER) && scaled) {
        if (bf16) {
            gather_mx8_kernel<true><<<dim3(mf::quads * mf::col_tiles, lay.tmax), 256, 0, ctx->stream>>>(
                x_dev, L.hidden, count, plan);
        } else {
            gather_mx8_kernel<false><<<dim3(mf::quads * mf::col_tiles, lay.tmax), 256, 0, ctx->stream>>>(
                x_dev, L.hidden, count, plan);
        }
        TTL_LAUNCHED("gather_mx8_kernel");
    } else if (stages & TTL_PREFILL_GATHER) {
        const dim3 grid(mf::quads, lay.tmax);
        if (bf16) {
            gather_kernel<true, 1><<<grid, mf::col_tiles * 64, 0, ctx->stream>>>(x_dev, L.hidden, count, plan);
        } else if (f16x) {
            Plan p = plan;
            if (x_shift_dev) {
                p.token_shift = const_cast<int32_t *>(x_shift_dev);
            } else {
                const int rc = ttl::launch_row_shifts(ctx->stream, static_cast<const float *>(x_dev), L.hidden,
                                                      count, L.hidden, plan.token_shift);
                if (rc != TTL_OK) {
                    return rc;
                }
            }
            gather_kernel<false, 2, true><<<grid, mf::col_tiles * 64, 0, ctx->stream>>>(x_dev, L.hidden, count, p);
        } else {
            gather_kernel<false, 3><<<grid, mf::col_tiles * 64, 0, ctx->stream>>>(x_dev, L.hidden, count, plan);
        }
        TTL_LAUNCHED("gather_kernel");
    }
    if ((stages & (TTL_PREFILL_GATEUP | TTL_PREFILL_DOWN | TTL_PREFILL_COMBINE)) == 0) {
        return TTL_OK;
    }

    GateUpArgs g;
    g.gate_codes = L.gate->codes;
    g.gate_scales = L.gate->scales;
    g.up_codes = L.up->codes;
    g.up_scales = L.up->scales;
    g.gate_bias = L.gate_bias;
    g.up_bias = L.up_bias;
    g.rows = L.expert_hidden;
    g.tiles_per_expert = L.gate->tiles;
    g.plan = plan;
    // one launch per GEMM over the wide tiles and the narrow ones (at most one per expert)
    const dim3 gu_grid((L.expert_hidden + kGuRows - 1) / kGuRows, lay.tmax);
    if ((stages & TTL_PREFILL_GATEUP) && scaled) {
        mx8_gateup_kernel<<<gu_grid, kGuWaves * 64, 0, ctx->stream>>>(g);
        TTL_LAUNCHED("mx8_gateup_kernel");
    } else if (stages & TTL_PREFILL_GATEUP) {
        if (bf16 && f16h) {
            gateup_kernel<1, true><<<gu_grid, kGuWaves * 64, 0, ctx->stream>>>(g);
        } else if (bf16) {
            gateup_kernel<1, false><<<gu_grid, kGuWaves * 64, 0, ctx->stream>>>(g);
        } else if (f16x && f16h) {
            gateup_kernel<2, true, mf::f16x8><<<gu_grid, kGuWaves * 64, 0, ctx->stream>>>(g);
        } else if (f16x) {
            gateup_kernel<2, false, mf::f16x8><<<gu_grid, kGuWaves * 64, 0, ctx->stream>>>(g);
        } else if (f16h) {
            gateup_kernel<3, true><<<gu_grid, kGuWaves * 64, 0, ctx->stream>>>(g);
        } else {
            gateup_kernel<3, false><<<gu_grid, kGuWaves * 64, 0, ctx->stream>>>(g);
        }
        TTL_LAUNCHED("gateup_kernel");
    }

    MatmulArgs m;
    m.codes = L.down->codes;
    m.scales = L.down->scales;
    m.bias = L.down_bias;
    m.rows = L.hidden;
    m.tiles_per_expert = L.down->tiles;
    m.frags = plan.hb;
    m.tile_planes = kHiddenPlanes;
    m.plan = plan;
    m.out = plan.down;
    m.out_rows = 0;
    if ((stages & TTL_PREFILL_DOWN) && scaled) {
        mx8_matmul_kernel<false><<<dim3(L.hidden / kMmRows, lay.tmax), kMmWaves * 64, 0, ctx->stream>>>(m);
        TTL_LAUNCHED("mx8_matmul_kernel");
    } else if ((stages & TTL_PREFILL_DOWN) && f16h) {
        matmul_kernel<2, false, mf::f16x8, mf::kHiddenF16Shift>
            <<<dim3(L.hidden / kMmRows, lay.tmax), kMmWaves * 64, 0, ctx->stream>>>(m);
        TTL_LAUNCHED("matmul_kernel");
    } else if (stages & TTL_PREFILL_DOWN) {
        matmul_kernel<kHiddenPlanes, false><<<dim3(L.hidden / kMmRows, lay.tmax), kMmWaves * 64, 0, ctx->stream>>>(m);
        TTL_LAUNCHED("matmul_kernel");
    }
    if (stages & TTL_PREFILL_COMBINE) {
        combine_for(L.used, plan, count, L.hidden, residual_dev, out_dev, ctx->stream);
        TTL_LAUNCHED("combine_kernel");
    }
    return TTL_OK;
}

}  // namespace

extern "C" {

int ttl_moe_prefill_stages(ttl_ctx *ctx, const ttl_moe_layer *layer, const void *x_dev, int x_dtype,
                           uint32_t count, const int32_t *indices_dev, const float *weights_dev, float *out_dev,
                           void *workspace_dev, size_t workspace_bytes, uint32_t stages) {
    return moe_prefill_run(ctx, layer, x_dev, x_dtype, count, indices_dev, weights_dev, out_dev, workspace_dev,
                           workspace_bytes, stages, nullptr, nullptr);
}

int ttl_moe_prefill_intermediates(ttl_ctx *ctx, const ttl_moe_layer *layer, int x_dtype, uint32_t count,
                                  const void *workspace_dev, size_t workspace_bytes, float *hidden_dev,
                                  float *down_dev, uint8_t *hidden_scales_dev) {
    TTL_REQUIRE(ctx && layer && layer->down && workspace_dev && hidden_dev && down_dev, TTL_ERR_INVALID,
                "ttl_moe_prefill_intermediates: null argument");
    TTL_REQUIRE(x_dtype == TTL_DTYPE_F32 || x_dtype == TTL_DTYPE_BF16 || x_dtype == TTL_DTYPE_F32_AS_MXFP8 ||
                    x_dtype == TTL_DTYPE_BF16_AS_MXFP8,
                TTL_ERR_INVALID, "ttl_moe_prefill_intermediates: unknown x_dtype %d", x_dtype);
    TTL_REQUIRE(layer->hidden == uint32_t(mx::cols) && layer->expert_hidden == uint32_t(mx::cols), TTL_ERR_SHAPE,
                "ttl_moe_prefill_intermediates: hidden and expert_hidden must be %d", mx::cols);
    TTL_REQUIRE(layer->used >= 1 && layer->used <= kMaxUsed && layer->experts >= 1 && layer->experts <= kMaxExperts,
                TTL_ERR_SHAPE, "ttl_moe_prefill_intermediates: used must be 1..%u and experts 1..%u", kMaxUsed,
                kMaxExperts);
    TTL_REQUIRE(uint64_t(count) * layer->used <= kMaxEntries, TTL_ERR_SHAPE,
                "ttl_moe_prefill_intermediates: count * used above %u", kMaxEntries);
    TTL_REQUIRE((reinterpret_cast<uintptr_t>(workspace_dev) & 255) == 0, TTL_ERR_INVALID,
                "ttl_moe_prefill_intermediates: workspace must be 256-byte aligned");
    if (count == 0) {
        return TTL_OK;
    }
    const uint32_t pairs = count * layer->used;
    const bool scaled = x_dtype == TTL_DTYPE_F32_AS_MXFP8 || x_dtype == TTL_DTYPE_BF16_AS_MXFP8;
    const bool bf16 = x_dtype == TTL_DTYPE_BF16 || x_dtype == TTL_DTYPE_BF16_AS_MXFP8;
    const Layout lay = make_layout(pairs, layer->experts, (bf16 || scaled) ? 1 : 3, true, layer->hidden,
                                   x_dtype == TTL_DTYPE_F32 ? count : 0);
    TTL_REQUIRE(workspace_bytes >= lay.total, TTL_ERR_SHAPE,
                "ttl_moe_prefill_intermediates: workspace of %zu bytes, %zu needed for this count and x_dtype",
                workspace_bytes, lay.total);
    const Plan plan = plan_at(const_cast<void *>(workspace_dev), lay);
    if (scaled) {
        prefill_intermediates_kernel<true, false><<<pairs, 256, 0, ctx->stream>>>(plan, layer->hidden, hidden_dev,
                                                                                   down_dev, hidden_scales_dev);
    } else if (hidden_f16(*layer)) {
        prefill_intermediates_kernel<false, true><<<pairs, 256, 0, ctx->stream>>>(plan, layer->hidden, hidden_dev,
                                                                                   down_dev, hidden_scales_dev);
    } else {
        prefill_intermediates_kernel<false, false><<<pairs, 256, 0, ctx->stream>>>(plan, layer->hidden, hidden_dev,
                                                                                    down_dev, hidden_scales_dev);
    }
    TTL_LAUNCHED("prefill_intermediates_kernel");
    return TTL_OK;
}

int ttl_moe_prefill_experts(ttl_ctx *ctx, const ttl_moe_layer *layer, const void *x_dev, int x_dtype,
                            uint32_t count, const int32_t *indices_dev, const float *weights_dev, float *out_dev,
                            void *workspace_dev, size_t workspace_bytes) {
    return ttl_moe_prefill_stages(ctx, layer, x_dev, x_dtype, count, indices_dev, weights_dev, out_dev,
                                  workspace_dev, workspace_bytes, TTL_PREFILL_ALL);
}

size_t ttl_moe_prefill_batch_workspace_bytes(uint32_t count, uint32_t experts, uint32_t used) {
    const size_t routing = align256(ttl::router_scratch_bytes() * count) + 2 * align256(4ull * count * used);
    return routing + ttl_moe_prefill_workspace_bytes(count, experts, used, TTL_DTYPE_F32);
}

int ttl_moe_prefill_fused(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *x_dev, const int32_t *x_shift_dev,
                          const float *residual_dev, uint32_t count, float *out_dev, int32_t *indices_dev,
                          float *weights_dev, void *workspace_dev, size_t workspace_bytes) {
    TTL_REQUIRE(ctx && layer && x_dev && out_dev && workspace_dev, TTL_ERR_INVALID, "ttl_moe_prefill: null argument");
    TTL_REQUIRE(layer->gate && layer->up && layer->down, TTL_ERR_INVALID, "ttl_moe_prefill: null expert tensor");
    for (const ttl_mxfp4 *t : {layer->gate, layer->up, layer->down}) {
        const int rc = check_bf16_scales(t, -1, "ttl_moe_prefill");  // before the router launches
        if (rc != TTL_OK) {
            return rc;
        }
    }
    TTL_REQUIRE(!layer->input_norm, TTL_ERR_INVALID,
                "ttl_moe_prefill: x is the normalized MoE input (model.cpp:549-551); the layer's input_norm must be NULL");
    TTL_REQUIRE((reinterpret_cast<uintptr_t>(residual_dev) & 15) == 0, TTL_ERR_INVALID,
                "ttl_moe_prefill: the residual must be 16-byte aligned");
    TTL_REQUIRE(layer->used >= 1 && layer->used <= kMaxUsed, TTL_ERR_SHAPE, "ttl_moe_prefill: used must be 1..%u",
                kMaxUsed);
    TTL_REQUIRE(workspace_bytes >= ttl_moe_prefill_batch_workspace_bytes(count, layer->experts, layer->used),
                TTL_ERR_SHAPE, "ttl_moe_prefill: workspace of %zu bytes, %zu needed", workspace_bytes,
                ttl_moe_prefill_batch_workspace_bytes(count, layer->experts, layer->used));
    TTL_REQUIRE((reinterpret_cast<uintptr_t>(workspace_dev) & 255) == 0, TTL_ERR_INVALID,
                "ttl_moe_prefill: workspace must be 256-byte aligned");
    if (count == 0) {
        return TTL_OK;
    }
    uint8_t *w = static_cast<uint8_t *>(workspace_dev);
    void *scratch = w;
    w += align256(ttl::router_scratch_bytes() * count);
    int32_t *indices = reinterpret_cast<int32_t *>(w);
    w += align256(4ull * count * layer->used);
    float *weights = reinterpret_cast<float *>(w);
    w += align256(4ull * count * layer->used);
    const size_t rest = workspace_bytes - size_t(w - static_cast<uint8_t *>(workspace_dev));
    int rc = ttl::launch_router_batch(ctx, *layer, x_dev, count, scratch, indices_dev ? indices_dev : indices,
                                      weights_dev ? weights_dev : weights);
    if (rc != TTL_OK) {
        return rc;
    }
    return moe_prefill_run(ctx, layer, x_dev, TTL_DTYPE_F32, count, indices_dev ? indices_dev : indices,
                           weights_dev ? weights_dev : weights, out_dev, w, rest, TTL_PREFILL_ALL, x_shift_dev,
                           residual_dev);
}

int ttl_moe_prefill(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *x_dev, uint32_t count, float *out_dev,
                    int32_t *indices_dev, float *weights_dev, void *workspace_dev, size_t workspace_bytes) {
    return ttl_moe_prefill_fused(ctx, layer, x_dev, nullptr, nullptr, count, out_dev, indices_dev, weights_dev,
                                 workspace_dev, workspace_bytes);
}

}  // extern "C"
