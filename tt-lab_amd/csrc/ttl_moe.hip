// MoE decode for one token: router + top-k + softmax, gate/up matvecs with the
// clamped SwiGLU fused in, down matvecs, rank-ordered weighted combine.
// Reference: GptOssModel::moe (model.cpp:292-338).
//
// Router and top-k.  The reference sums each router row sequentially in f32
// (tensor.cpp:186-200), and the expert indices must match it exactly.  A
// parallel sum rounds differently, so router_rows_kernel computes every row
// exactly (products are exact in f64, sums kept in f64) together with a rigorous
// bound on how far the reference's sequential f32 sum can be from it:
//     |ref - exact| <= u * (sum_k |w_k x_k| + sum_k |S_k|),  u = 2^-24,
// where S_k is the exact partial sum after column k (each product and each
// addition rounds by at most u times its exact result).  route_workgroup() then
// ranks the exact values; when the top-k order and the k/k+1 boundary are
// separated by more than the bounds, the reference's selection sort provably
// returns the same indices.  Otherwise (and for any non-finite value) it
// recomputes every logit in the reference's sequential order and replays the
// reference's selection sort (model.cpp:296-309) on them.
//
// route_workgroup() runs in one workgroup after the rows are known and publishes
// indices, weights and logits; the gate/up kernel then reads the indices.
#include "ttl_moe_math.hpp"
#include "ttl_mxfp4_tile.hpp"
#include "ttl_stage.hpp"

#include <cmath>
#include <type_traits>
#include <utility>

namespace {

constexpr int kRouterThreads = 192;  // 180 lanes x 16 columns = 2880
constexpr int kRouterCols = 2880;
constexpr uint32_t kMaxExperts = 192;
constexpr uint32_t kMaxUsed = 16;
constexpr int kPerLane = kMaxExperts / 64;  // candidates per lane in the wave-wide selection

using moe_math::clamped_swiglu;
using moe_math::std_max;
using moe_math::std_min;

__device__ inline double wave_inclusive_scan(double v, uint32_t lane) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const double t = __shfl_up(v, d);
        if (lane >= uint32_t(d)) {
            v += t;
        }
    }
    return v;
}

__device__ inline double wave_sum(double v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        v += __shfl_xor(v, d);
    }
    return v;
}

// model.cpp:310-321: softmax over the selected logits in rank order (both arrays
// in LDS, so no per-thread array needs scratch memory).
__device__ void softmax_selected(const float *selected, uint32_t k, float *weights) {
#pragma clang fp contract(off)
    float maximum = -INFINITY;
    for (uint32_t i = 0; i < k; ++i) {
        maximum = std_max(maximum, selected[i]);
    }
    float sum = 0.0f;
    for (uint32_t i = 0; i < k; ++i) {
        weights[i] = expf(selected[i] - maximum);
        sum = sum + weights[i];
    }
    for (uint32_t i = 0; i < k; ++i) {
        weights[i] = weights[i] / sum;
    }
}

struct RouterScratch {
    double exact[kMaxExperts];  // exact logit (f64)
    double bound[kMaxExperts];  // bound on |reference - exact|
    uint32_t exact_path_count;
};

// One workgroup per router row of one token: the exact value of the row (f64) and
// the bound on the reference's sequential-sum error.  180 lanes hold 16 columns each.
template <int MODE>
__global__ __launch_bounds__(kRouterThreads) void router_rows_kernel(const float *__restrict__ weight,
                                                                     const float *__restrict__ bias,
                                                                     stage::Input in, RouterScratch *scratch,
                                                                     float *__restrict__ normed_out) {
    __shared__ double wave_part[3][3];
    __shared__ __attribute__((aligned(16))) float xs[mxt::x_floats];
    __shared__ float red[stage::red_floats(mxt::x_blocks)];
    const uint32_t row = blockIdx.x;
    const uint32_t t = threadIdx.x, lane = t % 64, wave = t / 64;
    const bool active = t < kRouterCols / 16;

    stage::Pending<kRouterCols, mxt::x_blocks, kRouterThreads, MODE> pending;
    stage::stage_load(in, pending);
    // unconditional (idle lanes re-read lane 179's columns): loads under a branch make
    // the compiler wait for them at its end, before the staging could overlap them
    float4 wv[4];
    const float4 *w4 = reinterpret_cast<const float4 *>(weight + size_t(row) * kRouterCols) +
                       4 * (active ? t : uint32_t(kRouterCols / 16 - 1));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        wv[q] = w4[q];
    }
    stage::stage_finish(in, pending, xs, red);
    // the workgroups hand the staged (normalized) input on, a slice each: the routed
    // gate/up launch stages it as it is instead of normalizing the same vector again in
    // each of its workgroups
    if (normed_out) {
        const uint32_t slice = (uint32_t(kRouterCols) + gridDim.x - 1) / gridDim.x;
        const uint32_t end = min(uint32_t(kRouterCols), (row + 1) * slice);
        for (uint32_t c = row * slice + t; c < end; c += kRouterThreads) {
            normed_out[c] = xs[(c / 32) * mxt::x_stride + c % 32];
        }
    }
    double prod[16];
    double local = 0.0, abs_sum = 0.0;
    if (active) {
        // lane t holds columns 16t .. 16t+15: half of block t/2 in the padded layout
        const float *xt = xs + (t / 2) * mxt::x_stride + (t % 2) * 16;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 w = wv[q], v = *reinterpret_cast<const float4 *>(xt + 4 * q);
            prod[4 * q + 0] = double(w.x) * double(v.x);
            prod[4 * q + 1] = double(w.y) * double(v.y);
            prod[4 * q + 2] = double(w.z) * double(v.z);
            prod[4 * q + 3] = double(w.w) * double(v.w);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            local += prod[i];
            abs_sum += fabs(prod[i]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            prod[i] = 0.0;
        }
    }
    // exclusive prefix of the per-lane sums across the 180 lanes
    const double incl = wave_inclusive_scan(local, lane);
    if (lane == 63) {
        wave_part[0][wave] = incl;
    }
    __syncthreads();
    double offset = incl - local;
    for (uint32_t w = 0; w < wave; ++w) {
        offset += wave_part[0][w];
    }
    const double b = double(bias[row]);
    double running = b + offset, partial_abs = 0.0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        running += prod[i];
        partial_abs += fabs(running);
    }
    if (!active) {
        partial_abs = 0.0;
    }
    const double s_abs = wave_sum(partial_abs), s_prod = wave_sum(abs_sum);
    if (lane == 0) {
        wave_part[1][wave] = s_abs;
        wave_part[2][wave] = s_prod;
    }
    __syncthreads();
    if (t == 0) {
        const double total = b + wave_part[0][0] + wave_part[0][1] + wave_part[0][2];
        const double abs_partials = wave_part[1][0] + wave_part[1][1] + wave_part[1][2];
        const double abs_products = wave_part[2][0] + wave_part[2][1] + wave_part[2][2];
        scratch->exact[row] = total;
        // u = 2^-24; 1.001 covers second-order terms (n u < 2e-4); the 1e-12 term
        // covers the f64 rounding of the exact sums; 1e-37 covers subnormal steps.
        scratch->bound[row] = 1.001 * 0x1p-24 * (abs_partials + abs_products) + 1e-12 * abs_products + 1e-37;
    }
}

// Routing result shared by a workgroup.
struct RouteLds {
    int32_t indices[kMaxUsed];
    float weights[kMaxUsed];
    float selected[kMaxUsed];
    float ref_logits[kMaxExperts];
    int32_t order[kMaxExperts];
    int certified;
};

__device__ inline double wave_max(double v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        v = fmax(v, __shfl_xor(v, d));
    }
    return v;
}

// Order-preserving key of a double: a > b (neither NaN) gives key(a) >= key(b),
// strictly for unequal values except -0.0 below +0.0.
__device__ inline uint64_t order_key(double v) {
    const uint64_t u = uint64_t(__double_as_longlong(v));
    return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

__device__ inline double key_value(uint64_t key) {
    return __longlong_as_double((key >> 63) ? (long long)(key & 0x7fffffffffffffffull) : (long long)(~key));
}

__device__ inline uint64_t readlane_u64(uint64_t x, uint32_t lane) {
    const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(x)), int(lane)));
    const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(x >> 32)), int(lane)));
    return (uint64_t(hi) << 32) | lo;
}

// max(x, x of the lane that the DPP pattern CTRL names); every pattern used stays
// inside a row of 16 lanes
template <int CTRL>
__device__ inline uint64_t max_dpp(uint64_t x) {
    const uint32_t lo = uint32_t(__builtin_amdgcn_update_dpp(0, int(uint32_t(x)), CTRL, 0xf, 0xf, false));
    const uint32_t hi = uint32_t(__builtin_amdgcn_update_dpp(0, int(uint32_t(x >> 32)), CTRL, 0xf, 0xf, false));
    const uint64_t y = (uint64_t(hi) << 32) | lo;
    return y > x ? y : x;
}

// Maximum over the 64 lanes of a wave (all lanes active); the result is uniform.
// Quad swaps, then the half-row and row mirrors leave each row's maximum in all
// its lanes; the four rows meet through lane reads.
__device__ inline uint64_t wave_max_u64(uint64_t x) {
    x = max_dpp<0xb1>(x);   // quad_perm [1,0,3,2]
    x = max_dpp<0x4e>(x);   // quad_perm [2,3,0,1]
    x = max_dpp<0x141>(x);  // row_half_mirror
    x = max_dpp<0x140>(x);  // row_mirror
    uint64_t m = readlane_u64(x, 0);
#pragma unroll
    for (uint32_t r = 1; r < 4; ++r) {
        const uint64_t y = readlane_u64(x, 16 * r);
        m = y > m ? y : m;
    }
    return m;
}

// Order-preserving key of a float: a > b (neither NaN) gives key(a) >= key(b),
// strictly for unequal values except -0.0 below +0.0.
__device__ inline uint32_t order_key32(float v) {
    const uint32_t u = __float_as_uint(v);
    return (u >> 31) ? ~u : (u | 0x80000000u);
}

// The 32-bit form of wave_max_u64: DPP within rows, then the four rows' lane reads.
__device__ inline uint32_t wave_max_u32(uint32_t x) {
    x = max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0xb1, 0xf, 0xf, false)));   // quad_perm [1,0,3,2]
    x = max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x4e, 0xf, 0xf, false)));   // quad_perm [2,3,0,1]
    x = max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x141, 0xf, 0xf, false)));  // row_half_mirror
    x = max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x140, 0xf, 0xf, false)));  // row_mirror
    const uint32_t a = uint32_t(__builtin_amdgcn_readlane(int(x), 0));
    const uint32_t b = uint32_t(__builtin_amdgcn_readlane(int(x), 16));
    const uint32_t c = uint32_t(__builtin_amdgcn_readlane(int(x), 32));
    const uint32_t d = uint32_t(__builtin_amdgcn_readlane(int(x), 48));
    return max(max(a, b), max(c, d));
}

// Routing for one token comes in two parts.  route_certified_wave() ranks the
// exact rows; when the ranking is certified it leaves the indices (and, when
// `publish`, the softmax weights and -- if `logits` is non-null, in one workgroup
// of a launch -- the logits) in lds with lds.certified = 1.  Otherwise (or with
// force_exact) an exact path recomputes the logits in the reference's order from
// the staged router input (the same values the router rows saw) and replays the
// reference's selection sort.  Both end with a workgroup barrier, so
// lds.certified is uniform.
//
// The ranking runs in wave 0 alone, in registers.  Thread c < experts would rank
// expert c by (exact value descending, index ascending) -- the order the
// reference's selection sort produces when no two values are within their error
// bounds.  Lane l holds experts l, l+64, l+128.  A candidate's key is the 32-bit
// order key of its exact value rounded to f32: one wave maximum per rank gives the
// largest key, and a ballot picks the lowest expert holding it.  The rounding only
// merges values the certificate rejects anyway: two values with one f32 image are
// less than one f32 ulp apart, and each bound is at least half an ulp of its value
// (2^-24 of the sum of |products|), so they are never separated by their bounds.
// The certificate compares the exact values and bounds, value - bound of rank r >
// value + bound of every expert ranked below r, which holds only if the values are
// strictly ordered as ranked (bounds are positive).  Checked as
// up(r') < min(low of ranks before r') at each rank and max(up of the unselected)
// < min(low of all selected) at the end.  Leaves indices, selected values and
// lds.certified (and, when `publish`, weights and logits) in lds; ends with the
// workgroup's one barrier.
// Wave 0's share of the router rows (exact values and bounds), loaded ahead of
// route_certified_wave() so a caller can issue the loads before others.
// PL candidates per lane (lane l holds experts l, l + 64, ...), at most kPerLane: the
// decode launch picks the smallest PL that holds the layer's experts, so the loops over
// a lane's candidates are as short as the expert count allows.
template <int PL = kPerLane>
struct RouteRows {
    double v[PL], b[PL];
};

template <int PL>
__device__ __forceinline__ void load_route_rows(uint32_t experts, const RouterScratch *scratch, RouteRows<PL> &rows) {
    if (threadIdx.x < 64) {
#pragma unroll
        for (int j = 0; j < PL; ++j) {
            const uint32_t c = threadIdx.x + 64 * j;
            rows.v[j] = c < experts ? scratch->exact[c] : 0.0;
            rows.b[j] = c < experts ? scratch->bound[c] : 0.0;
        }
    }
}

template <int PL>
__device__ void route_certified_wave(uint32_t experts, uint32_t k, bool force_exact, const RouteRows<PL> &rows,
                                     RouteLds &lds, float *__restrict__ logits, bool publish) {
    if (threadIdx.x < 64) {
        const uint32_t lane = threadIdx.x;
        uint32_t key[PL];
        double low[PL], up[PL];
        float value[PL];
        bool bad = false;
#pragma unroll
        for (int j = 0; j < PL; ++j) {
            const uint32_t c = lane + 64 * j;
            key[j] = 0;
            low[j] = 0.0;
            up[j] = -INFINITY;
            value[j] = 0.0f;
            if (c < experts) {
                const double v = rows.v[j], b = rows.b[j];
                bad = bad || !isfinite(v) || !isfinite(b);
                key[j] = order_key32(float(v));
                low[j] = v - b;
                up[j] = v + b;
                value[j] = float(v);
            }
        }
        bool ok = !force_exact && __ballot(bad) == 0;
        double min_low = INFINITY;
        for (uint32_t r = 0; r < k; ++r) {
            uint32_t m = key[0];
#pragma unroll
            for (int j = 1; j < PL; ++j) {
                m = max(m, key[j]);
            }
            m = wave_max_u32(m);
            // the lowest expert holding the largest key (candidates are numbered lane +
            // 64 j, so the first piece with a match, then its lowest lane)
            uint32_t c = ~0u;
#pragma unroll
            for (int j = PL - 1; j >= 0; --j) {
                const uint64_t hit = __ballot(key[j] == m && m != 0u);
                if (hit) {
                    c = 64u * uint32_t(j) + uint32_t(__ffsll((long long)hit) - 1);
                }
            }
            c = c == ~0u ? 0u : c;
            const uint32_t owner = c % 64, piece = c / 64;
            double lo_c = low[0], up_c = up[0];
            float v_c = value[0];
#pragma unroll
            for (int j = 1; j < PL; ++j) {
                if (piece == uint32_t(j)) {
                    lo_c = low[j];
                    up_c = up[j];
                    v_c = value[j];
                }
            }
            const double w_low = __longlong_as_double((long long)readlane_u64(uint64_t(__double_as_longlong(lo_c)), owner));
            const double w_up = __longlong_as_double((long long)readlane_u64(uint64_t(__double_as_longlong(up_c)), owner));
            const float w_v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v_c), int(owner)));
#pragma unroll
            for (int j = 0; j < PL; ++j) {
                if (lane + 64 * j == c) {
                    key[j] = 0;
                    up[j] = -INFINITY;
                }
            }
            ok = ok && (r == 0 || w_up < min_low);
            min_low = fmin(min_low, w_low);
            if (lane == 0) {
                lds.indices[r] = int32_t(c);
                lds.selected[r] = w_v;
            }
        }
        uint64_t u = order_key(up[0]);
#pragma unroll
        for (int j = 1; j < PL; ++j) {
            const uint64_t y = order_key(up[j]);
            u = y > u ? y : u;
        }
        ok = ok && min_low > key_value(wave_max_u64(u));
        if (lane == 0) {
            lds.certified = ok ? 1 : 0;
            if (ok && publish) {
                softmax_selected(lds.selected, k, lds.weights);
            }
        }
        if (ok && publish && logits) {
#pragma unroll
            for (int j = 0; j < PL; ++j) {
                if (lane + 64 * j < experts) {
                    logits[lane + 64 * j] = value[j];
                }
            }
        }
    }
    __syncthreads();
}

// The reference's selection sort (model.cpp:296-309) replayed on lds.ref_logits, then
// the softmax of the selected logits.  Wave 0 only; ends with a barrier.
__device__ __forceinline__ void replay_selection(uint32_t experts, uint32_t k, RouterScratch *scratch, RouteLds &lds,
                                 bool count_exact) {
    const uint32_t t = threadIdx.x, lane = t % 64;
    if (t < 64) {
        // one step per rank: best starts at position i and moves to j only if
        // value[j] > value[best].  So best stays at i when value[order[i]] is NaN, and
        // otherwise is the first position >= i holding the largest non-NaN value.
        for (uint32_t i = 0; i < k; ++i) {
            const bool start_nan = isnan(lds.ref_logits[lds.order[i]]);
            double m = -INFINITY;
#pragma unroll
            for (int j = 0; j < kPerLane; ++j) {
                const uint32_t p = lane + 64 * j;
                if (p >= i && p < experts) {
                    const float val = lds.ref_logits[lds.order[p]];
                    if (!isnan(val)) {
                        m = fmax(m, double(val));
                    }
                }
            }
            m = wave_max(m);
            int32_t best = 0x7fffffff;
#pragma unroll
            for (int j = 0; j < kPerLane; ++j) {
                const uint32_t p = lane + 64 * j;
                if (p >= i && p < experts && double(lds.ref_logits[lds.order[p]]) == m) {
                    best = min(best, int32_t(p));
                }
            }
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) {
                best = min(best, __shfl_xor(best, d));
            }
            if (start_nan) {
                best = int32_t(i);
            }
            if (lane == 0) {
                const int32_t tmp = lds.order[i];
                lds.order[i] = lds.order[best];
                lds.order[best] = tmp;
                lds.indices[i] = lds.order[i];
            }
            // lane 0's LDS swap must land before the wave reads order[] again
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        if (lane == 0) {
            for (uint32_t r = 0; r < k; ++r) {
                lds.selected[r] = lds.ref_logits[lds.indices[r]];
            }
            softmax_selected(lds.selected, k, lds.weights);
            if (count_exact) {
                scratch->exact_path_count += 1;
            }
        }
    }
    __syncthreads();
}

// The exact path inside the routed gate/up kernel: thread t < experts forms row t's
// logit in the reference's order, sum = bias, then sum = sum + w[c] * x[c] for c =
// 0..2879 (tensor.cpp:186-200), from the staged router input xs.  Few registers, so
// the gate/up kernel keeps its occupancy; it runs for about 0.4% of decode tokens.
__device__ void route_exact_serial(const float *__restrict__ weight, const float *__restrict__ bias,
                                   uint32_t experts, uint32_t k, const float *xs, RouterScratch *scratch,
                                   RouteLds &lds, float *__restrict__ logits) {
    const uint32_t t = threadIdx.x;
    if (t < experts) {
#pragma clang fp contract(off)
        const float *w = weight + size_t(t) * kRouterCols;
        float sum = bias[t];
        for (int c = 0; c < kRouterCols; ++c) {
            sum = sum + w[c] * xs[(c / 32) * mxt::x_stride + c % 32];
        }
        lds.ref_logits[t] = sum;
        lds.order[t] = int32_t(t);
        if (logits) {
            logits[t] = sum;
        }
    }
    __syncthreads();
    replay_selection(experts, k, scratch, lds, logits != nullptr);
}

// The exact path of the standalone selection (a batch can hold many tokens and one
// uncertain token holds the whole launch, so its latency matters): the same sums, but
// the workgroup forms the products w[c] * x[c] (each rounded to f32, as the
// reference's) a tile of TC columns at a time into LDS, and thread t < experts only adds
// its row's products in column order.  The products of tile j + 1 are formed into the
// other of two LDS buffers while the adders sum tile j (one barrier per tile), and the
// adders read their row four products at a time.  Every thread holds 8 float4 pieces of
// each tile, loaded kAhead tiles before their products are formed (the router rows come
// from L2 or the MALL, about a microsecond away).  TC is chosen so a tile holds at most
// 7680 products (32 experts: 240 columns, 12 tiles; 128: 60; 192: 40).
template <int TC>
struct ExactTile {
    static constexpr int cols = TC;
    static constexpr int quads = TC / 4;                               // float4 pieces of one row's tile
    static constexpr int rows = 7680 / TC;                             // experts a tile holds
    static constexpr int stride = quads % 2 == 0 ? TC + 4 : TC + 8;    // floats; stride / 4 odd: the
                                                                       // adders' b128 reads miss each other's banks
    static constexpr int tiles = kRouterCols / TC;
    static constexpr int ahead = TC >= 240 ? 3 : 6;                    // tiles of loads in flight
    static constexpr int per = 8;                                      // pieces per thread (<= 2048 per tile)
    static constexpr int lds_floats = 2 * rows * stride;
    static_assert(kRouterCols % TC == 0 && tiles % ahead == 0, "whole tiles, whole rings");
    static_assert(rows * quads <= per * 256, "a tile's pieces fit the workgroup");
    static_assert((stride / 4) % 2 == 1 && stride % 4 == 0, "aligned rows, odd in float4");
};

template <int TC>
__device__ __forceinline__ void route_exact_coop(const float *__restrict__ weight, const float *__restrict__ bias,
                                                 uint32_t experts, uint32_t k, const float *xs,
                                                 RouterScratch *scratch, RouteLds &lds, float *__restrict__ logits,
                                                 float *prod) {
    using T = ExactTile<TC>;
    constexpr int PER = T::per, D = T::ahead;
    const uint32_t t = threadIdx.x;
    const uint32_t pieces = experts * T::quads;
    // piece i of a tile: expert i / quads, columns 4 (i % quads) .. + 3; pieces past the
    // tile's last re-read the last one (all loads unconditional) and are not stored
    auto piece = [&](int i) __attribute__((always_inline)) { return min(t + 256u * uint32_t(i), pieces - 1); };
    auto load = [&](int tile, float4(&r)[PER]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const uint32_t e = piece(i) / T::quads, c = uint32_t(tile) * TC + 4 * (piece(i) % T::quads);
            r[i] = *reinterpret_cast<const float4 *>(weight + size_t(e) * kRouterCols + c);
        }
    };
    // forms tile `tile`'s products into buffer tile % 2
    auto produce = [&](int tile, const float4(&r)[PER]) __attribute__((always_inline)) {
        float *buf = prod + (tile % 2) * (T::rows * T::stride);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
#pragma clang fp contract(off)
            const uint32_t e = piece(i) / T::quads, c4 = 4 * (piece(i) % T::quads);
            const uint32_t c = uint32_t(tile) * TC + c4;
            const float4 x = *reinterpret_cast<const float4 *>(xs + (c / 32) * mxt::x_stride + c % 32);
            if (t + 256u * uint32_t(i) < pieces) {
                const float4 w = r[i];
                *reinterpret_cast<float4 *>(buf + e * T::stride + c4) =
                    make_float4(w.x * x.x, w.y * x.y, w.z * x.z, w.w * x.w);
            }
        }
    };
    float4 wv[D][PER];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        load(d, wv[d]);
    }
    float sum = t < experts ? bias[t] : 0.0f;
    produce(0, wv[0]);
    load(D, wv[0]);
    __syncthreads();
#pragma unroll 1
    for (int base = 0; base < T::tiles; base += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int tile = base + d;
            const int next_slot = (d + 1) % D;  // a constant once the loop is unrolled
            if (tile + 1 < T::tiles) {
                produce(tile + 1, wv[next_slot]);
                // refill the slot (past the last tile: re-read it, unused)
                load(min(tile + 1 + D, T::tiles - 1), wv[next_slot]);
            }
            if (t < experts) {
                // chunks of kChunk float4: the next chunk's reads are issued before this
                // chunk's adds, so the LDS latency hides behind 4 kChunk dependent adds
                const float4 *row = reinterpret_cast<const float4 *>(prod + (tile % 2) * (T::rows * T::stride) +
                                                                     t * T::stride);
                constexpr int kChunk = T::quads % 12 == 0 ? 12 : (T::quads % 10 == 0 ? 10 : 5);
                constexpr int kChunks = T::quads / kChunk;
                static_assert(T::quads % kChunk == 0, "whole chunks");
                float4 pa[kChunk], pb[kChunk];
#pragma unroll
                for (int q = 0; q < kChunk; ++q) {
                    pa[q] = row[q];
                }
#pragma unroll
                for (int c = 0; c < kChunks; ++c) {
                    float4(&cur)[kChunk] = c % 2 == 0 ? pa : pb;
                    float4(&nxt)[kChunk] = c % 2 == 0 ? pb : pa;
                    if (c + 1 < kChunks) {
#pragma unroll
                        for (int q = 0; q < kChunk; ++q) {
                            nxt[q] = row[(c + 1) * kChunk + q];
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int q = 0; q < kChunk; ++q) {
#pragma clang fp contract(off)
                        sum = sum + cur[q].x;
                        sum = sum + cur[q].y;
                        sum = sum + cur[q].z;
                        sum = sum + cur[q].w;
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            __syncthreads();  // tile + 1 formed; the adders are done with tile's buffer
        }
    }
    if (t < experts) {
        lds.ref_logits[t] = sum;
        lds.order[t] = int32_t(t);
        if (logits) {
            logits[t] = sum;
        }
    }
    __syncthreads();
    replay_selection(experts, k, scratch, lds, logits != nullptr);
}

template <int MODE, int TC>
__device__ void route_workgroup(const float *__restrict__ weight, const float *__restrict__ bias,
                                const stage::Input &in, uint32_t experts, uint32_t k, bool force_exact,
                                RouterScratch *scratch, RouteLds &lds, float *__restrict__ logits, float *xs,
                                float *red, float *prod) {
    RouteRows<kPerLane> rows;
    load_route_rows<kPerLane>(experts, scratch, rows);
    route_certified_wave<kPerLane>(experts, k, force_exact, rows, lds, logits, true);
    if (!lds.certified) {
        stage::stage<kRouterCols, mxt::x_blocks, 256, MODE>(in, xs, red);
        route_exact_coop<TC>(weight, bias, experts, k, xs, scratch, lds, logits, prod);
    }
}

// Standalone routing (ttl_router_topk): one workgroup per token, publishes
// everything.  Workgroup t of a batch routes token t: input in.base + t * x_stride,
// scratch[t], outputs indices/weights_out + t * k (logits only for one token).
template <int MODE, int TC>
__global__ __launch_bounds__(256) void router_select_kernel(const float *__restrict__ weight,
                                                            const float *__restrict__ bias, uint32_t experts,
                                                            stage::Input in, uint32_t k, uint32_t force_exact,
                                                            RouterScratch *scratch, float *__restrict__ logits,
                                                            int32_t *__restrict__ indices,
                                                            float *__restrict__ weights_out, uint32_t x_stride) {
    __shared__ RouteLds lds;
    in.base += size_t(blockIdx.x) * x_stride;
    scratch += blockIdx.x;
    indices += size_t(blockIdx.x) * k;
    weights_out += size_t(blockIdx.x) * k;
    __shared__ __attribute__((aligned(16))) float xs[mxt::x_floats];
    __shared__ float red[stage::red_floats(mxt::x_blocks)];
    __shared__ __attribute__((aligned(16))) float prod[ExactTile<TC>::lds_floats];  // [2][rows][stride]
    route_workgroup<MODE, TC>(weight, bias, in, experts, k, force_exact != 0, scratch, lds, logits, xs, red,
                              prod);
    if (threadIdx.x < k) {
        indices[threadIdx.x] = lds.indices[threadIdx.x];
        weights_out[threadIdx.x] = lds.weights[threadIdx.x];
    }
}

// Router logits of a batch in the reference's own order (matmul_add_f32,
// tensor.cpp:498-527: sum = bias, then sum = sum + w[c] * x[c] for c = 0..2879,
// every product and every sum rounded to f32).  Each logit is one chain of 2880
// dependent adds, so a batch is as many chains as (token, expert) pairs: lane l of
// wave w runs token blockIdx.x * 64 + l against expert blockIdx.y * W + w.  The
// workgroup's 64 token rows are staged a tile of kRcCols columns at a time into one
// of two LDS buffers, the next tile's loads in flight while the waves run the
// current one (one barrier per tile); a lane reads its token's columns 16 bytes at
// a time.  The expert's weights reach the products through DPP: for each 64-column
// group g of the tile, lane l holds columns 64 g + 4 (l % 16) .. + 3 (each 16-lane
// row the same), and the product of column 64 g + 4 j + i takes component i from
// lane j of its row (row_newbcast), so the broadcast costs no instruction.  One wave
// per SIMD (W <= 4): a wave's two VALU operations per column (product, sum) are the
// chain's issue rate.  Logits go to logits[token * experts + expert]; past the
// batch or the experts, a lane reads a stand-in row and stores nothing.
constexpr int kRcTokens = 64;
constexpr int kRcGroups = 3;                 // 64-column groups per tile
constexpr int kRcCols = 64 * kRcGroups;      // 15 tiles
constexpr int kRcStride = kRcCols + 4;       // floats; stride / 4 odd: the lanes' b128 reads miss each other's banks
constexpr int kRcQuads = kRcCols / 4;
static_assert(kRouterCols % kRcCols == 0 && (kRcStride / 4) % 2 == 1, "whole tiles, conflict-free rows");

// lane j of the caller's 16-lane row (row_newbcast:j)
template <int J>
__device__ __forceinline__ float row_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + J, 0xf, 0xf, true));
}

// f(std::integral_constant<int, 0>) .. f(std::integral_constant<int, N - 1>), in order
template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <int W>
__global__ __launch_bounds__(64 * W) void router_chain_batch_kernel(const float *__restrict__ weight,
                                                                    const float *__restrict__ bias,
                                                                    const float *__restrict__ x, uint32_t x_stride,
                                                                    uint32_t count, uint32_t experts,
                                                                    float *__restrict__ logits) {
    constexpr int kTiles = kRouterCols / kRcCols;
    constexpr int kPer = kRcTokens * kRcQuads / (64 * W);  // token pieces (16 bytes) per thread and tile
    constexpr int kChunk = 4;                              // float4 of x per LDS read batch
    constexpr int kChunks = kRcQuads / kChunk;
    static_assert(kRcTokens * kRcQuads % (64 * W) == 0 && 16 % kChunk == 0, "whole pieces, chunks within a group");
    constexpr int kStaged = (kPer + kChunks - 1) / kChunks;  // staged pieces per chunk
    static_assert(kTiles % 2 == 1, "tile pairs, then the last tile");
    // a native vector (not HIP's float4 struct), so the staged pieces stay in registers
    typedef float f4 __attribute__((ext_vector_type(4)));
    __shared__ __attribute__((aligned(16))) float xs[2][kRcTokens * kRcStride];
    const uint32_t t = threadIdx.x, lane = t % 64;
    const uint32_t wave = uint32_t(__builtin_amdgcn_readfirstlane(int(t / 64)));
    const uint32_t token0 = blockIdx.x * kRcTokens;
    const uint32_t last = count - 1 - token0;  // the grid covers the batch: token0 < count
    const uint32_t expert = blockIdx.y * W + wave;
    const f4 *wsrc =
        reinterpret_cast<const f4 *>(weight + size_t(min(expert, experts - 1)) * kRouterCols) + lane % 16;
    // token piece i of a tile: token (t + 64 W i) / kRcQuads (clamped to the batch),
    // float4 (t + 64 W i) % kRcQuads
    const float *xg = x + size_t(token0) * x_stride;
    uint32_t src[kPer], dst[kPer];  // float offsets from xg, from the LDS buffer
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const uint32_t p = t + 64u * W * uint32_t(i);
        src[i] = min(p / kRcQuads, last) * x_stride + 4 * (p % kRcQuads);
        dst[i] = (p / kRcQuads) * kRcStride + 4 * (p % kRcQuads);
    }
    // Two register sets of a tile's token pieces: tile t + 1 is stored from set
    // (t + 1) % 2 at tile t, which then loads tile t + 3, so a tile's loads have two
    // tiles' time to land.  The weights are loaded a tile ahead.
    f4 ra[kPer], rb[kPer], wt[kRcGroups], wn[kRcGroups];
    auto load = [&](f4(&r)[kPer], int tile) __attribute__((always_inline)) {
        const float *xt = xg + min(tile, kTiles - 1) * kRcCols;  // past the last tile: a re-read, unused
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            r[i] = *reinterpret_cast<const f4 *>(xt + src[i]);
        }
    };
    auto load_w = [&](f4(&w)[kRcGroups], int tile) __attribute__((always_inline)) {
        tile = min(tile, kTiles - 1);
#pragma unroll
        for (int g = 0; g < kRcGroups; ++g) {
            w[g] = wsrc[tile * kRcQuads + 16 * g];
        }
    };
    auto store = [&](const f4(&r)[kPer], int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            *reinterpret_cast<f4 *>(xs[buf] + dst[i]) = r[i];
        }
    };
    load(ra, 0);
    load_w(wt, 0);
    store(ra, 0);
    load(rb, 1);
    load(ra, 2);
    float sum = bias[min(expert, experts - 1)];
    __syncthreads();
    // tile `tile` from LDS buffer tile % 2 with the weights in wt; before chunk c,
    // stage(i) for its kStaged pieces i (a staged piece's store and its next load,
    // spread over the tile so a wave never waits to issue a burst of loads)
    auto compute = [&](int buf, auto &&stage) __attribute__((always_inline)) {
        const f4 *row = reinterpret_cast<const f4 *>(xs[buf] + lane * kRcStride);
        f4 xa[kChunk], xb[kChunk];
#pragma unroll
        for (int q = 0; q < kChunk; ++q) {
            xa[q] = row[q];
        }
        static_for<kChunks>([&](auto cc) __attribute__((always_inline)) {
            constexpr int c = decltype(cc)::value;
            f4(&xc)[kChunk] = c % 2 == 0 ? xa : xb;
            f4(&xn)[kChunk] = c % 2 == 0 ? xb : xa;
            if constexpr (c + 1 < kChunks) {
#pragma unroll
                for (int q = 0; q < kChunk; ++q) {
                    xn[q] = row[(c + 1) * kChunk + q];
                }
            }
            static_for<kStaged>([&](auto kk) __attribute__((always_inline)) {
                constexpr int i = c * kStaged + decltype(kk)::value;
                if constexpr (i < kPer) {
                    stage(std::integral_constant<int, i>{});
                }
            });
            __builtin_amdgcn_sched_barrier(0);
            const f4 w = wt[c * kChunk / 16];
            static_for<kChunk>([&](auto kk) __attribute__((always_inline)) {
#pragma clang fp contract(off)
                constexpr int J = (c * kChunk) % 16 + decltype(kk)::value;
                const f4 xq = xc[decltype(kk)::value];
                const float p0 = row_bcast<J>(w.x) * xq.x, p1 = row_bcast<J>(w.y) * xq.y;
                const float p2 = row_bcast<J>(w.z) * xq.z, p3 = row_bcast<J>(w.w) * xq.w;
                sum = sum + p0;
                sum = sum + p1;
                sum = sum + p2;
                sum = sum + p3;
            });
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    // one tile: tile + 1 into LDS buffer (tile + 1) % 2 (last read before the previous
    // barrier) from the set S holding it, which then loads tile + 3; the weights of
    // tile + 1 are loaded meanwhile and move to wt after this tile's products
    auto step = [&](auto s_, int tile) __attribute__((always_inline)) {
        constexpr int S = decltype(s_)::value;  // (tile + 1) % 2
        f4(&r)[kPer] = S == 1 ? rb : ra;
        load_w(wn, tile + 1);
        const float *xt = xg + min(tile + 3, kTiles - 1) * kRcCols;  // past the last tile: a re-read, unused
        compute(S ^ 1, [&](auto i_) __attribute__((always_inline)) {
            constexpr int i = decltype(i_)::value;
            *reinterpret_cast<f4 *>(xs[S] + dst[i]) = r[i];
            r[i] = *reinterpret_cast<const f4 *>(xt + src[i]);
        });
#pragma unroll
        for (int g = 0; g < kRcGroups; ++g) {
            wt[g] = wn[g];
        }
        __syncthreads();  // every wave is done with buffer tile % 2 before it is refilled
    };
#pragma unroll 1
    for (int tile = 0; tile + 1 < kTiles; tile += 2) {
        step(std::integral_constant<int, 1>{}, tile);
        step(std::integral_constant<int, 0>{}, tile + 1);
    }
    compute((kTiles - 1) % 2, [](auto) {});
    if (lane <= last && expert < experts) {
        logits[size_t(token0 + lane) * experts + expert] = sum;
    }
}

// The reference's selection sort and softmax (model.cpp:350-377) on a batch's exact
// logits: one 64-thread workgroup per token.
__global__ __launch_bounds__(64) void router_select_logits_kernel(const float *__restrict__ logits,
                                                                  uint32_t experts, uint32_t k,
                                                                  int32_t *__restrict__ indices,
                                                                  float *__restrict__ weights_out) {
    __shared__ RouteLds lds;
    const float *row = logits + size_t(blockIdx.x) * experts;
    for (uint32_t c = threadIdx.x; c < experts; c += 64) {
        lds.ref_logits[c] = row[c];
        lds.order[c] = int32_t(c);
    }
    __syncthreads();
    replay_selection(experts, k, nullptr, lds, false);
    if (threadIdx.x < k) {
        indices[size_t(blockIdx.x) * k + threadIdx.x] = lds.indices[threadIdx.x];
        weights_out[size_t(blockIdx.x) * k + threadIdx.x] = lds.weights[threadIdx.x];
    }
}

// ---- gate/up + SwiGLU -------------------------------------------------------

// gate/up: one workgroup per (slot, 16-row tile); waves 0..3 split the gate
// tile's K range, waves 4..7 the up tile's, then the SwiGLU of the 16 rows.
constexpr int kSplit = 4;
constexpr int kGateUpThreads = 2 * kSplit * 64;
using GateUpSplit = mxt::Split<kSplit>;

// Row `row` of a split-K tile: the waves' partial sums in wave order.
template <int W>
__device__ inline float sum_parts(const float (*part)[mx::tile_rows], uint32_t row) {
    float sum = part[0][row];
#pragma unroll
    for (int k = 1; k < W; ++k) {
        sum += part[k][row];
    }
    return sum;
}

struct GateUpArgs {
    const uint8_t *gate_codes, *gate_scales;
    const float *gate_bias;
    const uint8_t *up_codes, *up_scales;
    const float *up_bias;
    uint32_t rows, tiles, experts, k;
    stage::Input in;  // the layer input (optionally the residual stream + norm)
    const int32_t *expert_ids;
    float *hidden;
    // ROUTE: the selection from the router rows (expert_ids unused); workgroup 0
    // publishes indices, weights and logits
    const float *router_weight, *router_bias;
    RouterScratch *scratch;
    int32_t *indices_out;
    float *weights_out, *logits_out;
};

// ROUTE: every workgroup ranks the router rows itself (route_certified_wave in
// wave 0, or the exact fallback when the ranking is not certified) instead of
// reading a separate selection kernel's indices; the input loads are in flight
// meanwhile.
template <int MODE, bool ROUTE, int PL = kPerLane>
__global__ __launch_bounds__(kGateUpThreads) void gateup_swiglu_kernel(GateUpArgs a) {
    __shared__ __attribute__((aligned(16))) float xs[GateUpSplit::x_floats];
    __shared__ float red[stage::red_floats(GateUpSplit::x_blocks)];
    __shared__ float part[2][kSplit][mx::tile_rows];
    const uint32_t slot = blockIdx.x / a.tiles, tile = blockIdx.x % a.tiles;
    const uint32_t wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const uint32_t which = wave / kSplit, w = wave % kSplit;  // which: 0 gate, 1 up

    // input loads first (they depend on nothing), then the expert's weight loads;
    // the staging completes while those are in flight
    // ROUTE: wave 0's router rows first (the ranking waits for them, and loads
    // return in order), then the input loads, then the ranking
    RouteRows<PL> rows;
    if constexpr (ROUTE) {
        load_route_rows<PL>(a.experts, a.scratch, rows);
    }
    stage::Pending<mx::cols, GateUpSplit::x_blocks, kGateUpThreads, MODE> pending;
    stage::stage_load(a.in, pending);
    int32_t e;
    bool staged = false;
    if constexpr (ROUTE) {
        __shared__ RouteLds rl;
        // workgroup 0 publishes the routing; the others only need the indices
        const bool first = blockIdx.x == 0;
        float *logits = first ? a.logits_out : nullptr;
        route_certified_wave<PL>(a.experts, a.k, false, rows, rl, logits, first);
        if (!rl.certified) {
            // rare: the exact path needs the staged input first
            stage::stage_finish(a.in, pending, xs, red);
            route_exact_serial(a.router_weight, a.router_bias, a.experts, a.k, xs, a.scratch, rl, logits);
            staged = true;
        }
        e = rl.indices[slot];
        if (first && threadIdx.x < a.k) {
            a.indices_out[threadIdx.x] = rl.indices[threadIdx.x];
            a.weights_out[threadIdx.x] = rl.weights[threadIdx.x];
        }
    } else {
        e = a.expert_ids[slot];
    }
    // All weight loads are unconditional (an invalid expert reads expert 0 and its
    // output becomes NaN below): loads under a branch make the compiler wait for
    // every load at the branch's end.
    const bool valid = e >= 0 && uint32_t(e) < a.experts;
    const uint32_t e_safe = valid ? uint32_t(e) : 0u;
    const uint32_t row = tile * mx::tile_rows + lane % mx::tile_rows;
    const size_t brow = size_t(e_safe) * a.rows + row;
    const float gb = a.gate_bias ? a.gate_bias[brow] : 0.0f;
    const float ub = a.up_bias ? a.up_bias[brow] : 0.0f;
    mxt::SplitRegs<kSplit> regs;
    mxt::split_load<kSplit>(which == 0 ? a.gate_codes : a.up_codes, which == 0 ? a.gate_scales : a.up_scales,
                            size_t(e_safe) * a.tiles + tile, w, lane, regs);
    if (!staged) {
        stage::stage_finish(a.in, pending, xs, red);
    }
    const float acc = mxt::split_compute<kSplit>(regs, xs, w, lane);
    if (lane < mx::tile_rows) {
        part[which][w][lane] = acc;
    }
    __syncthreads();
    if (threadIdx.x < mx::tile_rows) {
        const float g = sum_parts<kSplit>(part[0], threadIdx.x), u = sum_parts<kSplit>(part[1], threadIdx.x);
        a.hidden[size_t(slot) * a.rows + row] =
            valid ? clamped_swiglu(a.gate_bias ? g + gb : g, a.up_bias ? u + ub : u) : __builtin_nanf("");
    }
}

// ---- down matvec (per-slot input) -------------------------------------------

// one workgroup per (slot, 16-row tile), its four waves splitting K
__global__ __launch_bounds__(kSplit * 64) void down_kernel(
    const uint8_t *__restrict__ codes, const uint8_t *__restrict__ scales, const float *__restrict__ bias,
    uint32_t rows, uint32_t tiles, uint32_t experts, const float *__restrict__ hidden, uint32_t hidden_stride,
    const int32_t *__restrict__ expert_ids, float *__restrict__ down) {
    __shared__ __attribute__((aligned(16))) float xs[GateUpSplit::x_floats];
    __shared__ float red[stage::red_floats(GateUpSplit::x_blocks)];
    __shared__ float part[kSplit][mx::tile_rows];
    const uint32_t slot = blockIdx.x / tiles, tile = blockIdx.x % tiles;
    const uint32_t w = threadIdx.x / 64, lane = threadIdx.x % 64;
    // the slot's input first, then the (unconditional) weight loads
    stage::Input in{};
    in.base = hidden + size_t(slot) * hidden_stride;
    stage::Pending<mx::cols, GateUpSplit::x_blocks, kSplit * 64, stage::kPlain> pending;
    stage::stage_load(in, pending);
    const int32_t e = expert_ids[slot];
    const bool valid = e >= 0 && uint32_t(e) < experts;
    const uint32_t e_safe = valid ? uint32_t(e) : 0u;
    const uint32_t row = tile * mx::tile_rows + lane % mx::tile_rows;
    const float b = bias ? bias[size_t(e_safe) * rows + row] : 0.0f;
    mxt::SplitRegs<kSplit> regs;
    mxt::split_load<kSplit>(codes, scales, size_t(e_safe) * tiles + tile, w, lane, regs);
    stage::stage_finish(in, pending, xs, red);
    const float acc = mxt::split_compute<kSplit>(regs, xs, w, lane);
    if (lane < mx::tile_rows) {
        part[w][lane] = acc;
    }
    __syncthreads();
    if (threadIdx.x < mx::tile_rows) {
        const float sum = sum_parts<kSplit>(part, threadIdx.x);
        down[size_t(slot) * rows + row] = !valid ? __builtin_nanf("") : (bias ? sum + b : sum);
    }
}

// ---- gate/up + SwiGLU and down in one launch (the decode step) -----------------------
//
// Workgroup (slot, tile) runs gateup_swiglu_kernel's work for its 16 hidden rows, then
// the down rows of the same tile index for the same slot.  Down needs all 2880 hidden
// values of its slot, written by the slot's 180 gate/up tiles, so the tiles hand them
// over inside the launch:
//  - a gate/up tile writes its 16 values into its own 128-byte mailbox line with
//    agent-scope stores (written through to the memory side), waits until they are
//    complete (s_waitcnt), then raises its flag in 8 replicas, one per XCD, each in a
//    line of its own: the launch's epoch, one more than the tile's flag of the launch
//    before (every launch runs every tile, so the tiles agree on it without a count);
//  - every workgroup issues its down tile's weight loads as soon as its gate/up work
//    is done (they depend only on the routing), then polls its slot's 180 flags in its
//    own XCD's replica, one lane each, boundedly, and reads the mailbox with ordinary
//    loads: no mailbox line is in an L2 when a launch starts (kernel boundaries write
//    the L2s back and invalidate them) and each line has one writer whose values are in
//    memory before its flag, so the first reader on an XCD fetches a line and the others
//    find it in that XCD's L2.
// No release or acquire fence: on this chip an agent-scope release writes back the
// XCD's whole L2 and an acquire invalidates it.  Every workgroup must be resident at
// once (a waiting workgroup holds its CU); the host launches this form only when the
// occupancy allows the whole grid, and a wait that reaches its bound counts a give-up
// and leaves NaN rows instead of hanging.  The down rows are split over the 8 waves
// (3 iterations each; down_kernel splits 4 ways): the same products in another order.
// Measured on config 3 (MI355X), graph replays: 16.7 us per launch against 10.5 + 5.8 us
// for gateup_swiglu_kernel and down_kernel, and the decode step 1.207 against 1.193 ms
// per token with it, so the step keeps the two launches.  Per-workgroup timestamps
// (s_memrealtime): every workgroup resident within 0.5 us, the gate/up tiles done at
// 5.4-10.2 us, each slot's waiters released 0.5-2.8 us after its last tile, the mailbox
// staged about 1 us later and the down rows 1 us after that (the last at 13.7 us).
// Earlier forms and what they cost: one arrival count per slot, polled by all 180 of
// the slot's workgroups and read past the L2, 46.8 us (the waiters saw the full count
// one after another, about 90 ns apart: accesses that bypass the L2 serialize on the
// line they share); the same with eight count lines per slot and the hidden read
// through the L2 after an agent-scope acquire (which invalidates the XCD's L2, once per
// workgroup), about 30 us; per-XCD flags with a global count of departed workgroups to
// advance the epoch, 22.7 us (720 atomics on one line at the end of every launch).
constexpr unsigned kHandoffSpinLimit = 1u << 21;
constexpr int kDownPer = 3;  // down iterations per wave: 8 x 3 = 24 >= 23
static_assert(kDownPer * 2 * kSplit * mx::lanes_k <= GateUpSplit::x_blocks, "the staged hidden covers the split");

constexpr uint32_t kHoMaxTiles = 180;  // 16-row tiles of a 2880-row gate/up matrix
constexpr uint32_t kHoXcds = 8;        // one flag replica per XCD (workgroup b runs on XCD b % 8)

struct Handoff {
    // per (slot, XCD, gate/up tile), one 128-byte line each: the launch in which the tile
    // published its hidden values (a consumer on XCD x polls replica x only, so each line
    // has the slot's waiters of one XCD, not all of them)
    uint32_t flags[kMaxUsed][kHoXcds][kHoMaxTiles][32];
    // per (slot, tile), one 128-byte line each: the tile's 16 hidden values (one writer
    // per line, so an XCD's L2 holds no part of another workgroup's line)
    float mailbox[kMaxUsed][kHoMaxTiles][32];
    uint32_t give_ups;  // waits that ended at the spin limit (their rows are NaN)
};

struct DownArgs {
    const uint8_t *codes, *scales;
    const float *bias;
    uint32_t rows, tiles;  // down rows (the hidden size) and their 16-row tiles
    float *down;           // [used][rows]
    Handoff *handoff;
};

template <int MODE, bool ROUTE, int PL = kPerLane>
__global__ __launch_bounds__(kGateUpThreads) void gateup_down_kernel(GateUpArgs a, DownArgs d) {
    __shared__ __attribute__((aligned(16))) float xs[GateUpSplit::x_floats];
    __shared__ float red[stage::red_floats(GateUpSplit::x_blocks)];
    __shared__ float part[2 * kSplit][mx::tile_rows];
    __shared__ int waited;
    const uint32_t slot = blockIdx.x / a.tiles, tile = blockIdx.x % a.tiles;
    const uint32_t wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const uint32_t which = wave / kSplit, w = wave % kSplit;  // which: 0 gate, 1 up

    // ---- gate/up + SwiGLU, as gateup_swiglu_kernel ----
    RouteRows<PL> rows;
    if constexpr (ROUTE) {
        load_route_rows<PL>(a.experts, a.scratch, rows);
    }
    stage::Pending<mx::cols, GateUpSplit::x_blocks, kGateUpThreads, MODE> pending;
    stage::stage_load(a.in, pending);
    int32_t e;
    bool staged = false;
    if constexpr (ROUTE) {
        __shared__ RouteLds rl;
        const bool first = blockIdx.x == 0;
        float *logits = first ? a.logits_out : nullptr;
        route_certified_wave<PL>(a.experts, a.k, false, rows, rl, logits, first);
        if (!rl.certified) {
            stage::stage_finish(a.in, pending, xs, red);
            route_exact_serial(a.router_weight, a.router_bias, a.experts, a.k, xs, a.scratch, rl, logits);
            staged = true;
        }
        e = rl.indices[slot];
        if (first && threadIdx.x < a.k) {
            a.indices_out[threadIdx.x] = rl.indices[threadIdx.x];
            a.weights_out[threadIdx.x] = rl.weights[threadIdx.x];
        }
    } else {
        e = a.expert_ids[slot];
    }
    const bool valid = e >= 0 && uint32_t(e) < a.experts;
    const uint32_t e_safe = valid ? uint32_t(e) : 0u;
    const uint32_t row = tile * mx::tile_rows + lane % mx::tile_rows;
    const size_t brow = size_t(e_safe) * a.rows + row;
    const float gb = a.gate_bias ? a.gate_bias[brow] : 0.0f;
    const float ub = a.up_bias ? a.up_bias[brow] : 0.0f;
    uint32_t epoch;
    {
        mxt::SplitRegs<kSplit> regs;
        mxt::split_load<kSplit>(which == 0 ? a.gate_codes : a.up_codes, which == 0 ? a.gate_scales : a.up_scales,
                                size_t(e_safe) * a.tiles + tile, w, lane, regs);
        // the launch's epoch: one more than the value this (slot, tile) published in the
        // launch before, which every tile of the slot also published (each launch runs all
        // of them), so no workgroup counts the launches for the others (720 atomics on one
        // line at the end of a launch took about 7 us); requested once the weight loads
        // are, as it is first needed at the end of gate/up
        epoch = __hip_atomic_load(&d.handoff->flags[slot][0][tile][0], __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT) + 1u;
        if (!staged) {
            stage::stage_finish(a.in, pending, xs, red);
        }
        const float acc = mxt::split_compute<kSplit>(regs, xs, w, lane);
        if (lane < mx::tile_rows) {
            part[which * kSplit + w][lane] = acc;
        }
    }
    __syncthreads();
    if (wave == 0) {
        if (lane < mx::tile_rows) {
            const float g = sum_parts<kSplit>(part, lane), u = sum_parts<kSplit>(part + kSplit, lane);
            const float h =
                valid ? clamped_swiglu(a.gate_bias ? g + gb : g, a.up_bias ? u + ub : u) : __builtin_nanf("");
            a.hidden[size_t(slot) * a.rows + row] = h;  // the caller's copy (read after the launch)
            __hip_atomic_store(&d.handoff->mailbox[slot][tile][lane], h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // the mailbox stores are this wave's: once they are complete, raise the tile's
        // flag in every XCD's replica
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (lane < kHoXcds) {
            __hip_atomic_store(&d.handoff->flags[slot][lane][tile][0], epoch, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }

    // ---- down: the weight loads first, then the wait for the slot's hidden ----
    const uint32_t kl = lane / mx::tile_rows;
    const size_t dtile = size_t(e_safe) * d.tiles + tile;
    const uint32_t drow = tile * mx::tile_rows + lane % mx::tile_rows;
    const float db = d.bias ? d.bias[size_t(e_safe) * d.rows + drow] : 0.0f;
    uint4 q[kDownPer];
    uint32_t sc[kDownPer];
    {
        const uint8_t *rec = d.scales + dtile * mx::tile_scale_bytes + size_t(lane) * mx::scale_pad;
        const uint4 *tc = reinterpret_cast<const uint4 *>(d.codes) + dtile * mx::blocks * mx::tile_rows +
                          lane % mx::tile_rows;
#pragma unroll
        for (int j = 0; j < kDownPer; ++j) {
            sc[j] = rec[wave * kDownPer + j];  // iteration 23: the record's pad byte (scale 2^0)
        }
#pragma unroll
        for (int j = 0; j < kDownPer; ++j) {
            const uint32_t kb = min(uint32_t(4 * (wave * kDownPer + j)) + kl, uint32_t(mx::blocks - 1));
            q[j] = ttl::load_stream(tc + size_t(kb) * mx::tile_rows);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (threadIdx.x == 0) {
        waited = 1;
    }
    __syncthreads();
    // one lane per gate/up tile of the slot polls its flag in this XCD's replica
    if (threadIdx.x < a.tiles) {
        const uint32_t *flag = &d.handoff->flags[slot][blockIdx.x % kHoXcds][threadIdx.x][0];
        unsigned spins = 0;
        while (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != epoch &&
               spins < kHandoffSpinLimit) {
            __builtin_amdgcn_s_sleep(1);
            ++spins;
        }
        if (spins == kHandoffSpinLimit) {
            waited = 0;  // gave up: counted below, never waits longer
        }
    }
    __syncthreads();
    // the slot's hidden from the mailbox, into the padded layout (blocks 90.. zero), with
    // ordinary loads: no part of a mailbox line is in any L2 at the start of a launch
    // (kernel boundaries write the L2s back and invalidate them) and each line has one
    // writer, whose values are in memory before its flag, so the first reader on an XCD
    // fetches the line from memory and the others find it in that XCD's L2.  All of a
    // thread's loads are requested before the first is used.
    const float(*mb)[32] = d.handoff->mailbox[slot];
    constexpr uint32_t kStaged = uint32_t(GateUpSplit::x_blocks) * 32;
    constexpr int kHiddenPer = int((kStaged + kGateUpThreads - 1) / kGateUpThreads);
    float hv[kHiddenPer];
#pragma unroll
    for (int k = 0; k < kHiddenPer; ++k) {
        const uint32_t i = min(threadIdx.x + uint32_t(k) * kGateUpThreads, uint32_t(mx::cols) - 1);
        hv[k] = mb[i / mx::tile_rows][i % mx::tile_rows];
    }
#pragma unroll
    for (int k = 0; k < kHiddenPer; ++k) {
        const uint32_t i = threadIdx.x + uint32_t(k) * kGateUpThreads;
        if (i < kStaged) {
            xs[(i / 32) * mxt::x_stride + i % 32] = i < uint32_t(mx::cols) ? hv[k] : 0.0f;
        }
    }
    __syncthreads();
    {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < kDownPer; ++j) {
            const uint32_t kb = 4 * (wave * kDownPer + j) + kl;
            acc += __builtin_amdgcn_ldexpf(mxt::block_dot(q[j], xs + kb * mxt::x_stride), int(sc[j]) - 127);
        }
        acc += __shfl_xor(acc, 16);
        acc += __shfl_xor(acc, 32);
        if (lane < mx::tile_rows) {
            part[wave][lane] = acc;
        }
    }
    __syncthreads();
    if (threadIdx.x < mx::tile_rows) {
        const float sum = sum_parts<2 * kSplit>(part, threadIdx.x);
        d.down[size_t(slot) * d.rows + drow] =
            (!valid || !waited) ? __builtin_nanf("") : (d.bias ? sum + db : sum);
    }
    if (threadIdx.x == 0) {
        if (!waited) {
            __hip_atomic_fetch_add(&d.handoff->give_ups, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// down + combine + residual for used == 4: one workgroup per 16-row tile holds all
// four slots (16 waves: slot = wave / 4, K split over wave % 4), so it can finish
// the rows: out = residual + (0 + w_0 d_0 + w_1 d_1 + w_2 d_2 + w_3 d_3), the
// reference's combine order (model.cpp:323-337) and residual add (model.cpp:592-594).
constexpr int kDcSlots = 4;
constexpr int kDcThreads = kDcSlots * kSplit * 64;

__global__ __launch_bounds__(kDcThreads) void down_combine_kernel(
    const uint8_t *__restrict__ codes, const uint8_t *__restrict__ scales, const float *__restrict__ bias,
    uint32_t rows, uint32_t tiles, uint32_t experts, const float *__restrict__ hidden, uint32_t hidden_stride,
    const int32_t *__restrict__ expert_ids, const float *__restrict__ weights, const float *__restrict__ residual,
    float *__restrict__ out, float *__restrict__ down_out) {
#pragma clang fp contract(off)
    constexpr int kGroups = GateUpSplit::x_blocks * 8;                       // float4 groups per slot (padded)
    constexpr int kPer = (kDcSlots * kGroups + kDcThreads - 1) / kDcThreads;  // 3
    __shared__ __attribute__((aligned(16))) float xs[kDcSlots][GateUpSplit::x_floats];
    __shared__ float part[kDcSlots][kSplit][mx::tile_rows];
    const uint32_t tile = blockIdx.x;
    const uint32_t wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const uint32_t slot = wave / kSplit, w = wave % kSplit;
    const uint32_t row = tile * mx::tile_rows + lane % mx::tile_rows;

    // the four slots' inputs first (groups past the row end re-read group 0)
    float4 hv[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const uint32_t f = threadIdx.x + uint32_t(k) * kDcThreads;
        const uint32_t sl = f / kGroups, g = f % kGroups;
        const bool inside = f < uint32_t(kDcSlots * kGroups) && g < uint32_t(mx::blocks * 8);
        hv[k] = reinterpret_cast<const float4 *>(hidden + size_t(inside ? sl : 0) * hidden_stride)[inside ? g : 0];
    }
    // epilogue operands (threads < 16 finish the rows), then the weight loads
    int32_t e[kDcSlots];
    float b[kDcSlots], wr[kDcSlots];
#pragma unroll
    for (int r = 0; r < kDcSlots; ++r) {
        e[r] = expert_ids[r];
        wr[r] = weights[r];
        const uint32_t er = (e[r] >= 0 && uint32_t(e[r]) < experts) ? uint32_t(e[r]) : 0u;
        b[r] = bias ? bias[size_t(er) * rows + row] : 0.0f;
    }
    const float res = residual ? residual[row] : 0.0f;
    const int32_t my_e = e[0] * (slot == 0) + e[1] * (slot == 1) + e[2] * (slot == 2) + e[3] * (slot == 3);
    const uint32_t e_safe = (my_e >= 0 && uint32_t(my_e) < experts) ? uint32_t(my_e) : 0u;
    mxt::SplitRegs<kSplit> regs;
    mxt::split_load<kSplit>(codes, scales, size_t(e_safe) * tiles + tile, w, lane, regs);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const uint32_t f = threadIdx.x + uint32_t(k) * kDcThreads;
        const uint32_t sl = f / kGroups, g = f % kGroups;
        if (f < uint32_t(kDcSlots * kGroups)) {
            const float4 v = g < uint32_t(mx::blocks * 8) ? hv[k] : make_float4(0.f, 0.f, 0.f, 0.f);
            *reinterpret_cast<float4 *>(&xs[sl][(g / 8) * mxt::x_stride + (g % 8) * 4]) = v;
        }
    }
    __syncthreads();
    const float acc = mxt::split_compute<kSplit>(regs, xs[slot], w, lane);
    if (lane < mx::tile_rows) {
        part[slot][w][lane] = acc;
    }
    __syncthreads();
    if (threadIdx.x < mx::tile_rows) {
        float m = 0.0f;
#pragma unroll
        for (int r = 0; r < kDcSlots; ++r) {
            float d = sum_parts<kSplit>(part[r], threadIdx.x);
            d = bias ? d + b[r] : d;
            if (!(e[r] >= 0 && uint32_t(e[r]) < experts)) {
                d = __builtin_nanf("");
            }
            if (down_out) {
                down_out[size_t(r) * rows + row] = d;
            }
            m = m + wr[r] * d;
        }
        out[row] = residual ? res + m : m;
    }
}

// model.cpp:323-337: out = 0; out += w_r * down_r for r = 0..k-1 (unfused).
__global__ void combine_kernel(const float *__restrict__ down, const float *__restrict__ weights, uint32_t k,
                               uint32_t n, const float *__restrict__ residual, float *__restrict__ out) {
#pragma clang fp contract(off)
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) {
        return;
    }
    float acc = 0.0f;
    for (uint32_t r = 0; r < k; ++r) {
        acc = acc + weights[r] * down[size_t(r) * n + i];
    }
    out[i] = residual ? residual[i] + acc : acc;
}

}  // namespace

// ---- per-context MoE workspace ---------------------------------------------------

namespace ttl {

struct MoeWorkspace {
    RouterScratch router;
    float logits[kMaxExperts];
    int32_t indices[kMaxUsed];
    float weights[kMaxUsed];
    alignas(256) float normed[2880];  // the router rows' normalized input, for the routed gate/up
    alignas(256) float hidden[kMaxUsed * 2880];
    alignas(256) float down[kMaxUsed * 2880];
    alignas(256) Handoff handoff;  // gateup_down_kernel's counts (zero between launches)
};

size_t moe_workspace_bytes() {
    return sizeof(MoeWorkspace);
}

}  // namespace ttl

namespace {

ttl::MoeWorkspace *workspace(ttl_ctx *ctx) {
    return reinterpret_cast<ttl::MoeWorkspace *>(ctx->moe_workspace);
}

int check_router(const float *weight, const float *bias, uint32_t experts, uint32_t hidden, const float *x,
                 uint32_t k) {
    TTL_REQUIRE(weight && bias && x, TTL_ERR_INVALID, "router: null argument");
    TTL_REQUIRE(hidden == uint32_t(kRouterCols), TTL_ERR_SHAPE, "router: hidden must be %d", kRouterCols);
    TTL_REQUIRE(experts >= 1 && experts <= kMaxExperts, TTL_ERR_SHAPE, "router: experts must be 1..%u", kMaxExperts);
    TTL_REQUIRE(k >= 1 && k <= kMaxUsed && k <= experts, TTL_ERR_SHAPE, "router: k must be 1..%u and <= experts",
                kMaxUsed);
    TTL_REQUIRE(((uintptr_t)weight & 15) == 0 && ((uintptr_t)x & 15) == 0, TTL_ERR_INVALID,
                "router: weight and x must be 16-byte aligned");
    return TTL_OK;
}

int check_layer(const ttl_moe_layer *layer, const char *who) {
    TTL_REQUIRE(layer, TTL_ERR_INVALID, "%s: null layer", who);
    const ttl_moe_layer &L = *layer;
    TTL_REQUIRE(L.gate && L.up && L.down, TTL_ERR_INVALID, "%s: null expert tensor", who);
    TTL_REQUIRE(L.hidden == uint32_t(mx::cols) && L.expert_hidden == uint32_t(mx::cols), TTL_ERR_SHAPE,
                "%s: hidden and expert_hidden must be %d", who, mx::cols);
    TTL_REQUIRE(L.gate->rows == L.expert_hidden && L.up->rows == L.expert_hidden && L.down->rows == L.hidden,
                TTL_ERR_SHAPE, "%s: expert tensor rows do not match the layer", who);
    TTL_REQUIRE(L.gate->experts == L.experts && L.up->experts == L.experts && L.down->experts == L.experts,
                TTL_ERR_SHAPE, "%s: expert tensors must hold %u experts", who, L.experts);
    TTL_REQUIRE(L.used >= 1 && L.used <= kMaxUsed && L.used <= L.experts, TTL_ERR_SHAPE,
                "%s: used must be 1..%u", who, kMaxUsed);
    return TTL_OK;
}

// The MoE input as the staging sees it: x itself, or rms_norm(x) when the layer
// carries its input norm (x is then the residual stream).
stage::Input layer_input(const ttl_moe_layer &L, const float *x) {
    stage::Input in;
    in.base = x;
    in.add = nullptr;
    in.add_w = nullptr;
    in.add_k = 0;
    in.norm_w = L.input_norm;
    in.eps = L.input_norm_epsilon;
    in.v_out = nullptr;
    return in;
}

// Calls f(std::integral_constant<int, TC>) with the exact path's tile width for
// `experts` rows: 240 columns up to 32 experts, 60 up to 128, 40 up to 192.
template <typename F>
void with_tile_cols(uint32_t experts, F &&f) {
    static_assert(kMaxExperts <= uint32_t(ExactTile<40>::rows), "the narrowest tile holds every row");
    if (experts <= uint32_t(ExactTile<240>::rows)) {
        f(std::integral_constant<int, 240>{});
    } else if (experts <= uint32_t(ExactTile<60>::rows)) {
        f(std::integral_constant<int, 60>{});
    } else {
        f(std::integral_constant<int, 40>{});
    }
}

// Router + top-k + softmax: the exact rows and their bounds (one workgroup per
// expert), then the certified selection (one workgroup), which publishes indices,
// weights and logits.
void launch_router(ttl_ctx *ctx, const float *weight, const float *bias, uint32_t experts, uint32_t k,
                   const stage::Input &in, bool force_exact, float *logits, int32_t *indices, float *weights) {
    RouterScratch *scratch = &workspace(ctx)->router;
    stage::with_mode(in, [&](auto mode) {
        constexpr int M = decltype(mode)::value;
        router_rows_kernel<M><<<experts, kRouterThreads, 0, ctx->stream>>>(weight, bias, in, scratch, nullptr);
        with_tile_cols(experts, [&](auto tc) {
            router_select_kernel<M, decltype(tc)::value><<<1, 256, 0, ctx->stream>>>(
                weight, bias, experts, in, k, force_exact ? 1u : 0u, scratch, logits, indices, weights, 0u);
        });
    });
}

// The router rows alone (one workgroup per expert): the routed gate/up kernel
// does the selection.
void launch_router_rows(ttl_ctx *ctx, const ttl_moe_layer &L, const stage::Input &in) {
    RouterScratch *scratch = &workspace(ctx)->router;
    stage::with_mode(in, [&](auto mode) {
        router_rows_kernel<decltype(mode)::value><<<L.experts, kRouterThreads, 0, ctx->stream>>>(
            L.router_weight, L.router_bias, in, scratch, in.norm_w ? workspace(ctx)->normed : nullptr);
    });
}

}  // namespace

namespace ttl {

size_t router_scratch_bytes() {
    return sizeof(RouterScratch);
}

// Routing of `count` tokens at once (GptOssModel::moe_batch's router and top-k,
// model.cpp:341-377): token t's input is x + t * hidden (already normalized), its
// logits in the reference's order go to the scratch (count * experts floats), its
// indices and weights to indices/weights + t * used.  The logits are exact, so no
// certificate and no fallback: a batch costs the same whatever its ties.
int launch_router_batch(ttl_ctx *ctx, const ttl_moe_layer &L, const float *x, uint32_t count, void *scratch,
                        int32_t *indices, float *weights) {
    const int rc = check_router(L.router_weight, L.router_bias, L.experts, L.hidden, x, L.used);
    if (rc != TTL_OK) {
        return rc;
    }
    TTL_REQUIRE(count < 65536, TTL_ERR_SHAPE, "moe_batch router: at most 65535 tokens per call");
    TTL_REQUIRE(!L.input_norm, TTL_ERR_INVALID, "moe_batch router: x is the normalized router input");
    // the logits in the reference's order (the scratch holds count * experts floats),
    // then the selection
    static_assert(sizeof(RouterScratch) >= 4 * kMaxExperts, "a token's scratch holds its logits");
    float *logits = static_cast<float *>(scratch);
    constexpr int W = 4;
    router_chain_batch_kernel<W>
        <<<dim3((count + kRcTokens - 1) / kRcTokens, (L.experts + W - 1) / W), 64 * W, 0, ctx->stream>>>(
            L.router_weight, L.router_bias, x, L.hidden, count, L.experts, logits);
    router_select_logits_kernel<<<count, 64, 0, ctx->stream>>>(logits, L.experts, L.used, indices, weights);
    TTL_LAUNCHED("moe_batch router kernels");
    return TTL_OK;
}

}  // namespace ttl

namespace {

// gate/up of the experts in expert_ids, or (expert_ids == nullptr) of the experts
// the kernel selects itself from the router rows in the context's scratch, which
// it publishes to indices/weights.
int launch_gateup(ttl_ctx *ctx, const ttl_moe_layer &L, const float *x, const int32_t *expert_ids, float *hidden,
                  int32_t *indices = nullptr, float *weights = nullptr) {
    GateUpArgs a{};
    a.gate_codes = L.gate->codes;
    a.gate_scales = L.gate->scales;
    a.gate_bias = L.gate_bias;
    a.up_codes = L.up->codes;
    a.up_scales = L.up->scales;
    a.up_bias = L.up_bias;
    a.rows = L.expert_hidden;
    a.tiles = L.expert_hidden / mx::tile_rows;
    a.experts = L.experts;
    a.k = L.used;
    a.in = layer_input(L, x);
    if (!expert_ids && L.input_norm) {
        // routed: the router rows launch before this one left the normalized input in the
        // context's workspace (the same values: the staging's norm is order-fixed)
        a.in.base = workspace(ctx)->normed;
        a.in.norm_w = nullptr;
    }
    a.expert_ids = expert_ids;
    a.hidden = hidden;
    a.router_weight = L.router_weight;
    a.router_bias = L.router_bias;
    a.scratch = &workspace(ctx)->router;
    a.indices_out = indices;
    a.weights_out = weights;
    a.logits_out = workspace(ctx)->logits;
    stage::with_mode(a.in, [&](auto mode) {
        if (expert_ids) {
            gateup_swiglu_kernel<decltype(mode)::value, false>
                <<<a.tiles * L.used, kGateUpThreads, 0, ctx->stream>>>(a);
        } else if (L.experts <= 64) {
            gateup_swiglu_kernel<decltype(mode)::value, true, 1>
                <<<a.tiles * L.used, kGateUpThreads, 0, ctx->stream>>>(a);
        } else if (L.experts <= 128) {
            gateup_swiglu_kernel<decltype(mode)::value, true, 2>
                <<<a.tiles * L.used, kGateUpThreads, 0, ctx->stream>>>(a);
        } else {
            gateup_swiglu_kernel<decltype(mode)::value, true, kPerLane>
                <<<a.tiles * L.used, kGateUpThreads, 0, ctx->stream>>>(a);
        }
    });
    TTL_LAUNCHED("gateup_swiglu_kernel");
    return TTL_OK;
}

// The fused gate/up + down launch of the decode step: its grid (4 slots x 180 tiles of
// 512 threads) must be resident at once.  Returns false, launching nothing, when the
// occupancy does not allow that; the caller then runs gate/up and down as two launches.
template <class Kernel>
bool fits_resident(ttl_ctx *ctx, Kernel kernel, uint32_t grid) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kGateUpThreads, 0) != hipSuccess) {
        return false;
    }
    return uint64_t(per_cu) * uint64_t(ctx->compute_units) >= grid;
}

int launch_gateup_down(ttl_ctx *ctx, const ttl_moe_layer &L, const float *x, float *hidden, int32_t *indices,
                       float *weights, float *down, bool *fused) {
    GateUpArgs a{};
    a.gate_codes = L.gate->codes;
    a.gate_scales = L.gate->scales;
    a.gate_bias = L.gate_bias;
    a.up_codes = L.up->codes;
    a.up_scales = L.up->scales;
    a.up_bias = L.up_bias;
    a.rows = L.expert_hidden;
    a.tiles = L.expert_hidden / mx::tile_rows;
    a.experts = L.experts;
    a.k = L.used;
    a.in = layer_input(L, x);
    if (L.input_norm) {
        a.in.base = workspace(ctx)->normed;  // left there by the router rows launch
        a.in.norm_w = nullptr;
    }
    a.expert_ids = nullptr;
    a.hidden = hidden;
    a.router_weight = L.router_weight;
    a.router_bias = L.router_bias;
    a.scratch = &workspace(ctx)->router;
    a.indices_out = indices;
    a.weights_out = weights;
    a.logits_out = workspace(ctx)->logits;
    DownArgs d{};
    d.codes = L.down->codes;
    d.scales = L.down->scales;
    d.bias = L.down_bias;
    d.rows = L.hidden;
    d.tiles = L.hidden / mx::tile_rows;
    d.down = down;
    d.handoff = &workspace(ctx)->handoff;
    const uint32_t grid = a.tiles * L.used;
    *fused = false;
    // the tile index of gate/up and of down is the same (both 180), so one grid covers both
    if (d.tiles != a.tiles || a.tiles > kHoMaxTiles || L.used > kMaxUsed) {
        return TTL_OK;
    }
    stage::with_mode(a.in, [&](auto mode) {
        constexpr int M = decltype(mode)::value;
        auto go = [&](auto kernel) {
            if (fits_resident(ctx, kernel, grid)) {
                kernel<<<grid, kGateUpThreads, 0, ctx->stream>>>(a, d);
                *fused = true;
            }
        };
        if (L.experts <= 64) {
            go(gateup_down_kernel<M, true, 1>);
        } else if (L.experts <= 128) {
            go(gateup_down_kernel<M, true, 2>);
        } else {
            go(gateup_down_kernel<M, true, kPerLane>);
        }
    });
    TTL_LAUNCHED("gateup_down_kernel");
    return TTL_OK;
}

}  // namespace

extern "C" {

int ttl_router_topk(ttl_ctx *ctx, const float *weight_dev, const float *bias_dev, uint32_t experts, uint32_t hidden,
                    const float *x_dev, uint32_t k, uint32_t flags, float *logits_dev, int32_t *indices_dev,
                    float *weights_dev) {
    TTL_REQUIRE(ctx && logits_dev && indices_dev && weights_dev, TTL_ERR_INVALID, "ttl_router_topk: null argument");
    int rc = check_router(weight_dev, bias_dev, experts, hidden, x_dev, k);
    if (rc != TTL_OK) {
        return rc;
    }
    ttl_moe_layer plain{};
    launch_router(ctx, weight_dev, bias_dev, experts, k, layer_input(plain, x_dev), (flags & 1u) != 0, logits_dev,
                  indices_dev, weights_dev);
    TTL_LAUNCHED("router kernels");
    return TTL_OK;
}

int ttl_router_exact_count(ttl_ctx *ctx, uint64_t *count) {
    TTL_REQUIRE(ctx && count, TTL_ERR_INVALID, "ttl_router_exact_count: null argument");
    uint32_t value = 0;
    TTL_HIP(hipMemcpyAsync(&value, &workspace(ctx)->router.exact_path_count, sizeof(value), hipMemcpyDeviceToHost,
                           ctx->stream));
    TTL_HIP(hipStreamSynchronize(ctx->stream));
    *count = value;
    return TTL_OK;
}

int ttl_moe_gateup_swiglu(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *x_dev,
                          const int32_t *indices_dev, float *hidden_dev) {
    TTL_REQUIRE(ctx && x_dev && indices_dev && hidden_dev, TTL_ERR_INVALID, "ttl_moe_gateup_swiglu: null argument");
    int rc = check_layer(layer, "ttl_moe_gateup_swiglu");
    if (rc != TTL_OK) {
        return rc;
    }
    return launch_gateup(ctx, *layer, x_dev, indices_dev, hidden_dev);
}

int ttl_moe_down(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *hidden_dev, const int32_t *indices_dev,
                 float *down_dev) {
    TTL_REQUIRE(ctx && hidden_dev && indices_dev && down_dev, TTL_ERR_INVALID, "ttl_moe_down: null argument");
    int rc = check_layer(layer, "ttl_moe_down");
    if (rc != TTL_OK) {
        return rc;
    }
    const ttl_moe_layer &L = *layer;
    const uint32_t down_tiles = L.hidden / mx::tile_rows;
    down_kernel<<<down_tiles * L.used, kSplit * 64, 0, ctx->stream>>>(L.down->codes, L.down->scales, L.down_bias,
                                                                       L.hidden, down_tiles, L.experts, hidden_dev,
                                                                       L.expert_hidden, indices_dev, down_dev);
    TTL_LAUNCHED("down_kernel");
    return TTL_OK;
}

int ttl_moe_route_gateup_stages(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *x_dev, float *hidden_dev,
                                int32_t *indices_dev, float *weights_dev, uint32_t stages) {
    TTL_REQUIRE(ctx && x_dev && hidden_dev && indices_dev && weights_dev, TTL_ERR_INVALID,
                "ttl_moe_route_gateup: null argument");
    TTL_REQUIRE((stages & ~uint32_t(TTL_ROUTE_ALL)) == 0, TTL_ERR_INVALID,
                "ttl_moe_route_gateup_stages: unknown stage bits 0x%x", stages);
    int rc = check_layer(layer, "ttl_moe_route_gateup");
    if (rc != TTL_OK) {
        return rc;
    }
    const ttl_moe_layer &L = *layer;
    rc = check_router(L.router_weight, L.router_bias, L.experts, L.hidden, x_dev, L.used);
    if (rc != TTL_OK) {
        return rc;
    }
    if (stages & TTL_ROUTE_ROWS) {
        launch_router_rows(ctx, L, layer_input(L, x_dev));
        TTL_LAUNCHED("router_rows_kernel");
    }
    if (stages & TTL_ROUTE_GATEUP) {
        return launch_gateup(ctx, L, x_dev, nullptr, hidden_dev, indices_dev, weights_dev);
    }
    return TTL_OK;
}

int ttl_moe_route_gateup(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *x_dev, float *hidden_dev,
                         int32_t *indices_dev, float *weights_dev) {
    return ttl_moe_route_gateup_stages(ctx, layer, x_dev, hidden_dev, indices_dev, weights_dev, TTL_ROUTE_ALL);
}

int ttl_moe_route_gateup_down(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *x_dev, float *hidden_dev,
                              int32_t *indices_dev, float *weights_dev, float *down_dev, uint32_t stages) {
    TTL_REQUIRE(ctx && x_dev && hidden_dev && indices_dev && weights_dev && down_dev, TTL_ERR_INVALID,
                "ttl_moe_route_gateup_down: null argument");
    TTL_REQUIRE((stages & ~uint32_t(TTL_ROUTE_ROWS | TTL_ROUTE_GATEUP_DOWN)) == 0, TTL_ERR_INVALID,
                "ttl_moe_route_gateup_down: unknown stage bits 0x%x", stages);
    int rc = check_layer(layer, "ttl_moe_route_gateup_down");
    if (rc != TTL_OK) {
        return rc;
    }
    const ttl_moe_layer &L = *layer;
    rc = check_router(L.router_weight, L.router_bias, L.experts, L.hidden, x_dev, L.used);
    if (rc != TTL_OK) {
        return rc;
    }
    if (stages & TTL_ROUTE_ROWS) {
        launch_router_rows(ctx, L, layer_input(L, x_dev));
        TTL_LAUNCHED("router_rows_kernel");
    }
    if (stages & TTL_ROUTE_GATEUP_DOWN) {
        bool fused = false;
        rc = launch_gateup_down(ctx, L, x_dev, hidden_dev, indices_dev, weights_dev, down_dev, &fused);
        if (rc != TTL_OK || fused) {
            return rc;
        }
        // the grid cannot be resident at once: gate/up and down as two launches
        rc = launch_gateup(ctx, L, x_dev, nullptr, hidden_dev, indices_dev, weights_dev);
        if (rc == TTL_OK) {
            rc = ttl_moe_down(ctx, layer, hidden_dev, indices_dev, down_dev);
        }
    }
    return rc;
}

int ttl_moe_gateup_down_fused(ttl_ctx *ctx, const ttl_moe_layer *layer, int *fused) {
    TTL_REQUIRE(ctx && layer && fused, TTL_ERR_INVALID, "ttl_moe_gateup_down_fused: null argument");
    const uint32_t tiles = layer->expert_hidden / mx::tile_rows, grid = tiles * layer->used;
    const auto kernel = layer->experts <= 64    ? gateup_down_kernel<stage::kPlain, true, 1>
                        : layer->experts <= 128 ? gateup_down_kernel<stage::kPlain, true, 2>
                                                : gateup_down_kernel<stage::kPlain, true, kPerLane>;
    *fused = (layer->hidden == layer->expert_hidden && fits_resident(ctx, kernel, grid)) ? 1 : 0;
    return TTL_OK;
}

int ttl_moe_handoff_give_ups(ttl_ctx *ctx, uint64_t *count) {
    TTL_REQUIRE(ctx && count, TTL_ERR_INVALID, "ttl_moe_handoff_give_ups: null argument");
    uint32_t value = 0;
    TTL_HIP(hipMemcpyAsync(&value, &workspace(ctx)->handoff.give_ups, sizeof(value), hipMemcpyDeviceToHost,
                           ctx->stream));
    TTL_HIP(hipStreamSynchronize(ctx->stream));
    *count = value;
    return TTL_OK;
}

int ttl_moe_combine(ttl_ctx *ctx, const float *down_dev, const float *weights_dev, uint32_t k, uint32_t n,
                    float *out_dev) {
    TTL_REQUIRE(ctx && down_dev && weights_dev && out_dev, TTL_ERR_INVALID, "ttl_moe_combine: null argument");
    TTL_REQUIRE(k >= 1 && k <= kMaxUsed && n > 0, TTL_ERR_SHAPE, "ttl_moe_combine: bad k or n");
    combine_kernel<<<ttl::blocks_for(n, 256), 256, 0, ctx->stream>>>(down_dev, weights_dev, k, n, nullptr, out_dev);
    TTL_LAUNCHED("combine_kernel");
    return TTL_OK;
}

int ttl_moe_down_combine(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *hidden_dev,
                         const int32_t *indices_dev, const float *weights_dev, const float *residual_dev,
                         float *out_dev, float *down_dev) {
    TTL_REQUIRE(ctx && hidden_dev && indices_dev && weights_dev && out_dev, TTL_ERR_INVALID,
                "ttl_moe_down_combine: null argument");
    int rc = check_layer(layer, "ttl_moe_down_combine");
    if (rc != TTL_OK) {
        return rc;
    }
    const ttl_moe_layer &L = *layer;
    const uint32_t tiles = L.hidden / mx::tile_rows;
    if (L.used == uint32_t(kDcSlots)) {
        down_combine_kernel<<<tiles, kDcThreads, 0, ctx->stream>>>(
            L.down->codes, L.down->scales, L.down_bias, L.hidden, tiles, L.experts, hidden_dev, L.expert_hidden,
            indices_dev, weights_dev, residual_dev, out_dev, down_dev);
        TTL_LAUNCHED("down_combine_kernel");
        return TTL_OK;
    }
    // other expert counts: the down matvecs, then the combine
    float *down = down_dev ? down_dev : workspace(ctx)->down;
    rc = ttl_moe_down(ctx, layer, hidden_dev, indices_dev, down);
    if (rc != TTL_OK) {
        return rc;
    }
    combine_kernel<<<ttl::blocks_for(L.hidden, 256), 256, 0, ctx->stream>>>(down, weights_dev, L.used, L.hidden,
                                                                           residual_dev, out_dev);
    TTL_LAUNCHED("combine_kernel");
    return TTL_OK;
}

int ttl_moe_decode(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *x_dev, float *out_dev,
                   int32_t *indices_dev, float *weights_dev) {
    TTL_REQUIRE(ctx && x_dev && out_dev, TTL_ERR_INVALID, "ttl_moe_decode: null argument");
    int rc = check_layer(layer, "ttl_moe_decode");
    if (rc != TTL_OK) {
        return rc;
    }
    const ttl_moe_layer &L = *layer;
    rc = check_router(L.router_weight, L.router_bias, L.experts, L.hidden, x_dev, L.used);
    if (rc != TTL_OK) {
        return rc;
    }
    ttl::MoeWorkspace *ws = workspace(ctx);
    int32_t *indices = indices_dev ? indices_dev : ws->indices;
    float *weights = weights_dev ? weights_dev : ws->weights;
    launch_router_rows(ctx, L, layer_input(L, x_dev));
    TTL_LAUNCHED("router_rows_kernel");
    rc = launch_gateup(ctx, L, x_dev, nullptr, ws->hidden, indices, weights);
    if (rc == TTL_OK) {
        rc = ttl_moe_down_combine(ctx, layer, ws->hidden, indices, weights, nullptr, out_dev, nullptr);
    }
    return rc;
}

}  // extern "C"
