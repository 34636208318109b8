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

// ---- f16 operands (the prefill's hidden as two planes) ------------------------------------
//
// v_mfma_f32_16x16x32_f16 has the bf16 instruction's operand layout and rate.  Its uses
// here: f32 vectors as two f16 planes, each scaled by a power of two 2^k first, against
// weights decoded to f16 (MXFP4) or taken as f16 (Q8_0 codes, exact).  MXFP4 products stay
// exact where every E2M1 value times its E8M0 scale is a normal f16, E8M0
// f16_scale_min..f16_scale_max; the two planes hold 22 of a value's 24 bits (hi rounded to
// nearest, lo the rounded remainder).  The scale keeps hi within the f16 range and lo a
// normal f16 for values down to 2^-17 of the largest: the SwiGLU hidden, of magnitude at
// most 7 x 8 = 56 (the clamps of model.cpp:328-332), takes the fixed k = kHiddenF16Shift;
// a token row takes its own k = row_shift(max |x|), applied back to the GEMM's sums (a
// power of two, exact) before anything else (a bias) is added to them.

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// 0.5 x 2^(e-127) >= 2^-14 and 6 x 2^(e-127) <= 65504
constexpr uint32_t f16_scale_min = 114, f16_scale_max = 140;
// The hidden is scaled by 2^kHiddenF16Shift before its split (56 x 2^8 = 14336 < 65504), so
// its low plane stays a normal f16 down to |h| = 2^-11.
constexpr int kHiddenF16Shift = 8;

__device__ inline f32x4 mfma(const f16x8 &a, const f16x8 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// decode_step with f16 weights (exact for E8M0 f16_scale_min..f16_scale_max).
__device__ inline f16x8 decode_step_f16(uint32_t word, float scale) {
    const f16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(word, scale, 0);
    const f16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(word, scale, 1);
    const f16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(word, scale, 2);
    const f16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(word, scale, 3);
    return f16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// The decode of operand type V (bf16x8 or f16x8).
template <class V>
__device__ inline V decode_as(uint32_t word, float scale);
template <>
__device__ inline bf16x8 decode_as<bf16x8>(uint32_t word, float scale) {
    return decode_step(word, scale);
}
template <>
__device__ inline f16x8 decode_as<f16x8>(uint32_t word, float scale) {
    return decode_step_f16(word, scale);
}

// Two f16 planes of 8 f32 values times 2^shift, packed as the MFMA fragments are (value
// 2k in the low half of dword k).  A non-finite value stays in the first plane (a NaN a
// NaN) and the second is zero.
__device__ inline void split_f16x2(const float (&v)[8], int shift, uint4 (&out)[2]) {
    uint32_t hi[8], lo[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float s = __builtin_amdgcn_ldexpf(v[j], shift);
        const _Float16 h = _Float16(s);
        const _Float16 l = isfinite(s) ? _Float16(s - float(h)) : _Float16(0.0f);
        hi[j] = __builtin_bit_cast(uint16_t, h);
        lo[j] = __builtin_bit_cast(uint16_t, l);
    }
    out[0] = make_uint4(hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16), hi[4] | (hi[5] << 16), hi[6] | (hi[7] << 16));
    out[1] = make_uint4(lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16), lo[4] | (lo[5] << 16), lo[6] | (lo[7] << 16));
}

// The shift k of a token row whose largest finite magnitude is m: m x 2^k in [2^14, 2^15),
// so every finite value's hi plane is at most 32768 (< 65504) and the GEMM's sums of the
// scaled values stay far from the f32 range (k runs from -112 for m near 2^127 to 163 for
// m = 2^-149; consumers scale their sums back before adding anything unscaled, such as a
// bias).  0 for a row with no nonzero finite value.  Non-finite values are left out of m:
// they stay non-finite in hi.
__device__ inline int row_shift(float m) {
    // m = f x 2^e with f in [0.5, 1) (subnormal m included): m x 2^(15 - e) in [2^14, 2^15)
    return m > 0.0f ? 15 - __builtin_amdgcn_frexp_expf(m) : 0;
}

// The largest finite |x| of this lane's values (NaN and infinities left out).
__device__ inline float finite_max(float m, float x) {
    const float a = __builtin_fabsf(x);
    return a <= 3.40282347e38f ? __builtin_fmaxf(m, a) : m;
}

}  // namespace mf

// The scaled path: v_mfma_scale_f32_16x16x128_f8f6f4 with MXFP4 weights as A and
// MXFP8 (E4M3 + an E8M0 scale per 32 values) activations as B.
//
// Operand layout, measured on gfx950 (one wave, structured operands):
//  - A lane (row r, group g) holds 32 fp4 values, value v = nibble v of its 16 bytes;
//    here that is the repacked code chunk of MXFP4 block 4i+g of row r, so value v is
//    block element v/2 + 16 (v%2) (GGUF order: byte j = elements j and j+16).
//  - A value (g, v) meets B lane group 2 (g&1) + v/16, byte 16 (g>>1) + v%16 (B lane
//    (column n, group gb) holds 32 fp8 bytes).
//  - K-block g (the 32 values of A lane group g) is scaled by the A scale of lane
//    (r, g) and by the B scale of lane (n, g), whichever B lanes hold its values.
//  - D as in the other 16x16 MFMAs: lane l gets rows 4(l/16)..+3 of column l%16.
// So activation scale groups are the natural 32-element blocks, as for the weights;
// only the placement of the fp8 bytes is permuted.  The instruction's accumulation is
// not exact in f32: within a 32-element K-block the products are aligned to the
// block's largest and bits below 2^-13 of it are dropped (measured: 256 + 2^-5 kept,
// 256 + 2^-6 gives 256); block sums and the accumulator are added in f32.
namespace mx8 {

typedef int32_t i32x8 __attribute__((ext_vector_type(8)));

constexpr int lane_bytes = 32;                  // fp8 values per B lane
constexpr size_t frag_bytes = 64 * lane_bytes;  // one (quad, column tile) B fragment: 2 KiB
constexpr int scale_pad = 24;                   // scale bytes per (column tile, lane): quads 0..22 + 1
// One token tile's B operand for all of K: fragments [quad][column tile][lane][32 B],
// then scales [column tile][lane][scale_pad].
constexpr size_t tile_frag_bytes = size_t(mf::quads) * mf::col_tiles * frag_bytes;  // 188416
constexpr size_t tile_scale_bytes = size_t(mf::col_tiles) * 64 * scale_pad;         // 6144
constexpr size_t tile_bytes = tile_frag_bytes + tile_scale_bytes;
static_assert(tile_bytes <= mf::plane_bytes, "an MXFP8 tile fits one bf16 plane of the workspace");

// Block element held as value v of an A lane (and so of the B bytes it meets).
__host__ __device__ inline uint32_t element_of_value(uint32_t v) {
    return v / 2 + 16 * (v % 2);
}
// B placement of element e of K-block g: lane group and byte.
__host__ __device__ inline uint32_t b_group(uint32_t g, uint32_t e) {
    const uint32_t v = 2 * (e % 16) + e / 16;
    return 2 * (g & 1) + v / 16;
}
__host__ __device__ inline uint32_t b_byte(uint32_t g, uint32_t e) {
    const uint32_t v = 2 * (e % 16) + e / 16;
    return 16 * (g >> 1) + v % 16;
}

// E8M0 exponent X of a block whose largest magnitude is m (finite): the smallest X
// with m / 2^X <= 448, the E4M3 maximum, so no element saturates, but never below
// -127, the smallest scale E8M0 holds (byte 0).  m / 2^(e-8) = significand x 256
// exceeds 448 exactly when the significand exceeds 1.75.  Every block whose maximum is
// at most 448 x 2^-127 (f32 subnormals included) takes -127; without the floor those
// with maxima up to 1.75 x 2^-120 would get -128..-134, which the E8M0 byte cannot hold.
__device__ inline int block_exponent(float m) {
    const uint32_t u = __float_as_uint(m);
    const int e = int((u >> 23) & 0xffu);
    const int x = e - 127 - 8 + ((u & 0x7fffffu) > 0x600000u ? 1 : 0);
    return x < -127 ? -127 : x;
}

// OCP E4M3 of a value with |v| <= 448, rounded to nearest even: subnormals m x 2^-9
// (m = 8 carries into the smallest normal), normals (1 + m/8) x 2^(e-7).
__device__ inline uint32_t e4m3(float v) {
    const uint32_t sign = (__float_as_uint(v) >> 24) & 0x80u;
    const float a = fabsf(v);
    if (a < 0x1p-6f) {
        return sign | uint32_t(__builtin_rintf(a * 512.0f));
    }
    const uint32_t ua = __float_as_uint(a);
    const uint32_t r = ua + 0x7ffffu + ((ua >> 20) & 1u);
    return sign | ((((r >> 23) - 120u) << 3) | ((r >> 20) & 7u));
}
constexpr uint32_t e4m3_nan = 0x7fu;

__device__ inline float e4m3_value(uint32_t b) {
    const uint32_t e = (b >> 3) & 15u, m = b & 7u;
    const float mag = e == 0 ? float(m) * 0x1p-9f : __uint_as_float(((e + 120u) << 23) | (m << 20));
    return (b & 0x80u) ? -mag : mag;
}

// D += A B with A = one MXFP4 code chunk per lane (16 bytes) and its E8M0 scale, B = 32
// fp8 bytes per lane and the E8M0 scale of K-block (lane / 16).
__device__ inline mf::f32x4 mfma(const uint4 &a, const i32x8 &b, uint32_t scale_a, uint32_t scale_b,
                                 const mf::f32x4 &c) {
    const i32x8 av = {int32_t(a.x), int32_t(a.y), int32_t(a.z), int32_t(a.w), 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, b, c, 4, 0, 0, int32_t(scale_a), 0,
                                                            int32_t(scale_b));
}

}  // namespace mx8
