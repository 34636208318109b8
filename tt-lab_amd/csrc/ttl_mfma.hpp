// MFMA building blocks of the batched (prefill) MXFP4 kernels on gfx950.
//
// Operand fragments of v_mfma_f32_16x16x32_bf16 (D = A B + C, A 16x32, B 32x16):
//  - lane l holds 8 bf16 of A row l%16 and 8 bf16 of B column l%16, both for the
//    same 8 K indices, chosen by the lane group g = l/16;
//  - lane l receives D rows 4g..4g+3 of column l%16.
// Which 8 K indices a lane group holds is free as long as A and B agree.  Here
// they follow the repacked MXFP4 layout (ttl_internal.hpp): lane (r, g) of a wave
// holds the 16 code bytes of block 4i+g of row r for quad i (4 blocks = 128 K);
// MFMA step s (0..3) of the quad uses code dword s, and byte b of that dword gives
// element 2b (low nibble, K offset 4s+b in the block) and element 2b+1 (high
// nibble, K offset 4s+b+16).  Activation fragments are built in the same order.
#pragma once

#include "ttl_internal.hpp"

namespace mf {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int quads = mx::iters;          // 23 groups of 4 blocks along K = 2880 (blocks 90, 91 empty)
constexpr int steps = quads * 4;          // 92 MFMA K-steps of 32
constexpr int col_tiles = 4;              // 16-token column tiles per 64-slot token tile
constexpr int tile_slots = col_tiles * 16;
constexpr size_t frag_bytes = 64 * 16;    // one operand fragment: 64 lanes x 8 bf16
// One token tile's operand for all of K, one bf16 plane: [step][col tile][lane][8 bf16].
constexpr size_t plane_bytes = size_t(steps) * col_tiles * frag_bytes;  // 376832

__device__ inline f32x4 mfma(const bf16x8 &a, const bf16x8 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// E8M0 byte -> the f32 scale 2^(e-127) of the gfx950 conversion (E2M1 values are
// 0..6, half the reference's integer table, tensor.cpp:34-44).  e = 0 is the
// subnormal 2^-127 and e = 255 has no f32 value (infinity here); the conversion is
// exact for e = 1..254 only, so the entry points refuse tensors holding 0 or 255
// (ttl_mxfp4::edge_scales) before any kernel decodes them.
__device__ inline float e8m0_scale(uint32_t e) {
    return e ? __uint_as_float(e << 23) : 0x1p-127f;
}

// The 8 bf16 weights of MFMA step S for one lane: the 4 code bytes of `word`, each
// as (low nibble, high nibble), times `scale`.
__device__ inline bf16x8 decode_step(uint32_t word, float scale) {
    const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 0);
    const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 1);
    const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 2);
    const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 3);
    return bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

template <int S>
__device__ inline uint32_t dword(const uint4 &q) {
    static_assert(S >= 0 && S < 4, "dword index");
    return S == 0 ? q.x : (S == 1 ? q.y : (S == 2 ? q.z : q.w));
}

__device__ inline bf16x8 as_bf16x8(const uint4 &v) {
    return __builtin_bit_cast(bf16x8, v);
}
__device__ inline bf16x8 as_bf16x8v(const u32x4 &v) {
    return __builtin_bit_cast(bf16x8, v);
}

// Splits 8 f32 values into P bf16 planes (hi, mid, lo) whose sum is each value.
// Each plane is the remainder truncated to bf16 (its top 8 significant bits), and
// the f32 remainder after it is exact; three planes therefore reproduce all 24
// bits of a normal f32, and truncation never rounds a finite value to infinity.
// A non-finite value stays in the first plane (NaN kept a NaN) and the others are
// zero, so an infinity is not turned into inf - inf.
template <int P>
__device__ inline void split_planes(const float (&v)[8], uint4 (&out)[P]) {
    float r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        r[j] = v[j];
    }
#pragma unroll
    for (int p = 0; p < P; ++p) {
        uint32_t b[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t u = __float_as_uint(r[j]);
            const bool finite = (u & 0x7f800000u) != 0x7f800000u;
            const bool nan = (u & 0x7fffffffu) > 0x7f800000u;
            b[j] = (u >> 16) | (nan ? 0x40u : 0u);
            r[j] = finite ? r[j] - __uint_as_float(u & 0xffff0000u) : 0.0f;
        }
        out[p] = make_uint4(b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16));
    }
}

}  // namespace mf
