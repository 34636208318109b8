/*
 * ttlab_oracle.c -- CPU restatement of tt-lab's quantized decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see ttlab_oracle.h).  Citations are to the reference
 * tenstorrent/tt-lab sources.  Build flags mirror the reference's rules.py:6-11:
 * -O3 -ffp-contract=off -march=x86-64-v3.  Every "sum += a * b" below is an
 * unfused multiply then add, exactly as the reference's default bodies compute.
 */
#include "ttlab_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* formats                                                                   */
/* ------------------------------------------------------------------------- */

/* tensor.cpp:34 -- twice the E2M1 value of each nibble code; code 8 is +0. */
static const int8_t mxfp4_int[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

static float bits_to_f32(uint32_t bits) {
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint32_t f32_to_bits(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    return bits;
}

int orc_has_avx512(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw");
}

/* tensor.cpp:36-44: E8M0 exponent e -> 2^(e-128) built from its bit pattern:
 * the two smallest exponents are subnormal patterns, all others (e-1)<<23.
 * e = 255 therefore gives 2^127, never NaN. */
float orc_mxfp4_scale(uint8_t exponent) {
    uint32_t bits;
    if (exponent < 2) {
        bits = 0x00200000u << exponent;
    } else {
        bits = (uint32_t)(exponent - 1) << 23;
    }
    return bits_to_f32(bits);
}

int orc_mxfp4_int(uint8_t code) {
    return mxfp4_int[code & 15];
}

/* tensor.cpp:163-165 converts through _Float16; this is the exact IEEE binary16
 * to binary32 widening (NaNs come out quiet, as the x86 F16C conversion does). */
float orc_fp16_to_fp32(uint16_t half) {
    const uint32_t sign = (uint32_t)(half & 0x8000u) << 16;
    const uint32_t exponent = (half >> 10) & 0x1fu;
    const uint32_t mantissa = half & 0x3ffu;
    if (exponent == 0) {
        /* zero or subnormal: mantissa * 2^-24, exact in binary32 */
        const float magnitude = (float)mantissa * 0x1p-24f;
        return sign ? -magnitude : magnitude;
    }
    if (exponent == 31) {
        return bits_to_f32(sign | 0x7f800000u | (mantissa << 13) | (mantissa ? 0x00400000u : 0u));
    }
    return bits_to_f32(sign | ((exponent + 112u) << 23) | (mantissa << 13));
}

/* requant.cpp:311-316: round to nearest even on the upper 16 bits. */
uint16_t orc_fp32_to_bf16(float value) {
    uint32_t bits = f32_to_bits(value);
    const uint32_t lsb = (bits >> 16) & 1u;
    bits += 0x7fffu + lsb;
    return (uint16_t)(bits >> 16);
}

float orc_bf16_to_fp32(uint16_t bits) {
    return bits_to_f32((uint32_t)bits << 16);
}

/* tensor.cpp:62-71 builds weight[e][code] = scale(e) * float(int(code)); the
 * product is exact or overflows to infinity (e = 255 with |int| >= 2). */
static float mxfp4_weight(uint8_t exponent, uint8_t code) {
    return orc_mxfp4_scale(exponent) * (float)mxfp4_int[code & 15];
}

void orc_mxfp4_dequant_blocks(const uint8_t *blocks, size_t n, float *out) {
    for (size_t b = 0; b < n; ++b) {
        const uint8_t *source = blocks + b * 17;
        for (size_t i = 0; i < 16; ++i) {
            const uint8_t packed = source[1 + i];
            out[b * 32 + i] = mxfp4_weight(source[0], packed & 0x0f);
            out[b * 32 + 16 + i] = mxfp4_weight(source[0], packed >> 4);
        }
    }
}

/* tensor.cpp:136-157 */
int64_t orc_tensor_row_bytes(uint32_t type, uint64_t n) {
    switch (type) {
        case ORC_TYPE_F32:
            return (int64_t)(n * 4);
        case ORC_TYPE_BF16:
            return (int64_t)(n * 2);
        case ORC_TYPE_Q8_0:
            if (n % 32) {
                return -1;
            }
            return (int64_t)(n / 32 * 34);
        case ORC_TYPE_MXFP4:
            if (n % 32) {
                return -1;
            }
            return (int64_t)(n / 32 * 17);
        default:
            return -1;
    }
}

/* ------------------------------------------------------------------------- */
/* 16-lane helpers restating the reference's AVX-512 reduction orders        */
/* ------------------------------------------------------------------------- */

/* GCC's _mm512_reduce_add_ps (avx512fintrin.h, __MM512_REDUCE_OP): halves are
 * added lane-wise 16->8->4, then lanes {0,1}+{2,3}, then lane 0 + lane 1. */
static float reduce_tree16(const float *acc) {
    float t8[8], t4[4], t2[2];
    for (int i = 0; i < 8; ++i) {
        t8[i] = acc[i + 8] + acc[i];
    }
    for (int i = 0; i < 4; ++i) {
        t4[i] = t8[i + 4] + t8[i];
    }
    t2[0] = t4[0] + t4[2];
    t2[1] = t4[1] + t4[3];
    return t2[0] + t2[1];
}

/* tensor.cpp:86-92: reduce_f32x16 is a sequential sum from 0.0f. */
static float reduce_sequential16(const float *acc) {
    float sum = 0.0f;
    for (int i = 0; i < 16; ++i) {
        sum += acc[i];
    }
    return sum;
}

/* ------------------------------------------------------------------------- */
/* a3: MXFP4 matvec                                                          */
/* ------------------------------------------------------------------------- */

/* tensor.cpp:258-304 (default): per row, bias first, then for each block and
 * each byte i the low-nibble element i and then the high-nibble element i+16,
 * each an unfused multiply then add.  The reference interleaves four rows; the
 * per-row order is the same. */
static void mxfp4_matvec_default(const uint8_t *matrix, const float *bias, size_t rows, size_t cols,
                                 const float *input, float *output) {
    const size_t blocks = cols / 32;
    const size_t row_bytes = blocks * 17;
    for (size_t row = 0; row < rows; ++row) {
        const uint8_t *data = matrix + row * row_bytes;
        float sum = bias[row];
        for (size_t block = 0; block < blocks; ++block) {
            const uint8_t *source = data + block * 17;
            const uint8_t exponent = source[0];
            for (size_t i = 0; i < 16; ++i) {
                const uint8_t packed = source[1 + i];
                const float x0 = input[block * 32 + i];
                const float x1 = input[block * 32 + 16 + i];
                sum += mxfp4_weight(exponent, packed & 0x0f) * x0;
                sum += mxfp4_weight(exponent, packed >> 4) * x1;
            }
        }
        output[row] = sum;
    }
}

/* tensor.cpp:116-131,239-256 (v4), lane by lane: lane i keeps one accumulator;
 * per block it scales x by the block scale (rounded), then fuses
 * acc = fma(int_lo, x_i*s, acc) and acc = fma(int_hi, x_{i+16}*s, acc);
 * the row result is bias + the GCC tree reduction of the 16 lanes. */
static void mxfp4_matvec_v4(const uint8_t *matrix, const float *bias, size_t rows, size_t cols,
                            const float *input, float *output) {
    const size_t blocks = cols / 32;
    const size_t row_bytes = blocks * 17;
    for (size_t row = 0; row < rows; ++row) {
        const uint8_t *data = matrix + row * row_bytes;
        float acc[16] = {0};
        for (size_t block = 0; block < blocks; ++block) {
            const uint8_t *source = data + block * 17;
            const float scale = orc_mxfp4_scale(source[0]);
            for (size_t i = 0; i < 16; ++i) {
                const uint8_t packed = source[1 + i];
                const float x0 = input[block * 32 + i] * scale;
                const float x1 = input[block * 32 + 16 + i] * scale;
                acc[i] = fmaf((float)mxfp4_int[packed & 0x0f], x0, acc[i]);
                acc[i] = fmaf((float)mxfp4_int[packed >> 4], x1, acc[i]);
            }
        }
        output[row] = bias[row] + reduce_tree16(acc);
    }
}

/* The same v4 arithmetic with AVX-512 intrinsics, for CPU-baseline timing. */
__attribute__((target("avx512f,avx512bw"))) static void
mxfp4_matvec_v4_simd(const uint8_t *matrix, const float *bias, size_t rows, size_t cols, const float *input,
                     float *output) {
    const size_t blocks = cols / 32;
    const size_t row_bytes = blocks * 17;
    const __m128i table = _mm_loadu_si128((const __m128i *)mxfp4_int);
    const __m128i low_mask = _mm_set1_epi8(0x0f);
    for (size_t row = 0; row < rows; ++row) {
        const uint8_t *data = matrix + row * row_bytes;
        __m512 acc = _mm512_setzero_ps();
        for (size_t block = 0; block < blocks; ++block) {
            const uint8_t *source = data + block * 17;
            const __m128i packed = _mm_loadu_si128((const __m128i *)(source + 1));
            const __m128i codes_lo = _mm_and_si128(packed, low_mask);
            const __m128i codes_hi = _mm_and_si128(_mm_srli_epi16(packed, 4), low_mask);
            const __m512 w_lo = _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm_shuffle_epi8(table, codes_lo)));
            const __m512 w_hi = _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm_shuffle_epi8(table, codes_hi)));
            const __m512 scale = _mm512_set1_ps(orc_mxfp4_scale(source[0]));
            const __m512 x0 = _mm512_mul_ps(_mm512_loadu_ps(input + block * 32), scale);
            const __m512 x1 = _mm512_mul_ps(_mm512_loadu_ps(input + block * 32 + 16), scale);
            acc = _mm512_fmadd_ps(w_lo, x0, acc);
            acc = _mm512_fmadd_ps(w_hi, x1, acc);
        }
        output[row] = bias[row] + _mm512_reduce_add_ps(acc);
    }
}

void orc_matvec_add_mxfp4(const uint8_t *matrix, const float *bias, size_t rows, size_t cols,
                          const float *input, float *output, size_t expert, int body) {
    /* tensor.cpp:243-244: expert e starts e*rows rows into the tensor and its bias e*rows in. */
    const uint8_t *expert_data = matrix + expert * rows * (cols / 32 * 17);
    const float *expert_bias = bias + expert * rows;
    if (body == ORC_BODY_V4_SIMD && orc_has_avx512()) {
        mxfp4_matvec_v4_simd(expert_data, expert_bias, rows, cols, input, output);
    } else if (body == ORC_BODY_V4 || body == ORC_BODY_V4_SIMD) {
        mxfp4_matvec_v4(expert_data, expert_bias, rows, cols, input, output);
    } else {
        mxfp4_matvec_default(expert_data, expert_bias, rows, cols, input, output);
    }
}

/* ------------------------------------------------------------------------- */
/* a4: selected-token MXFP4 matmul                                           */
/* ------------------------------------------------------------------------- */

/* tensor.cpp:306-317 */
void orc_transpose_selected(size_t cols, const float *input, const size_t *tokens, size_t count,
                            float *transposed) {
    for (size_t s = 0; s < count; ++s) {
        const size_t token = tokens[s];
        for (size_t column = 0; column < cols; ++column) {
            transposed[column * count + s] = input[token * cols + column];
        }
    }
}

/* tensor.cpp:319-495.  Per (row, selected token) the accumulator starts at the
 * bias and walks (block, i, low then high).  default: weight = scale*int, then
 * unfused acc += weight*x.  v4: acc = fma(scale*int, x, acc).  The four-row
 * tiling and the 16-token masking do not change the per-(row, token) order.
 * Results scatter to output[tokens[t]*rows + row]; other rows stay untouched. */
void orc_matmul_add_mxfp4_selected_transposed(const uint8_t *matrix, const float *bias, size_t rows,
                                              size_t cols, const float *transposed, const size_t *tokens,
                                              size_t count, float *output, float *workspace, size_t expert,
                                              int body) {
    const size_t blocks = cols / 32;
    const size_t row_bytes = blocks * 17;
    const uint8_t *expert_data = matrix + expert * rows * row_bytes;
    const float *expert_bias = bias + expert * rows;
    const int fused = body != ORC_BODY_DEFAULT;
    for (size_t row = 0; row < rows; ++row) {
        const uint8_t *data = expert_data + row * row_bytes;
        for (size_t s = 0; s < count; ++s) {
            workspace[s] = expert_bias[row];
        }
        for (size_t block = 0; block < blocks; ++block) {
            const uint8_t *source = data + block * 17;
            const float scale = orc_mxfp4_scale(source[0]);
            for (size_t i = 0; i < 16; ++i) {
                const uint8_t packed = source[1 + i];
                const float weight_lo = scale * (float)mxfp4_int[packed & 0x0f];
                const float weight_hi = scale * (float)mxfp4_int[packed >> 4];
                const float *input_lo = transposed + (block * 32 + i) * count;
                const float *input_hi = transposed + (block * 32 + 16 + i) * count;
                for (size_t s = 0; s < count; ++s) {
                    if (fused) {
                        workspace[s] = fmaf(weight_lo, input_lo[s], workspace[s]);
                        workspace[s] = fmaf(weight_hi, input_hi[s], workspace[s]);
                    } else {
                        workspace[s] += weight_lo * input_lo[s];
                        workspace[s] += weight_hi * input_hi[s];
                    }
                }
            }
        }
        for (size_t t = 0; t < count; ++t) {
            output[tokens[t] * rows + row] = workspace[t];
        }
    }
}

/* ------------------------------------------------------------------------- */
/* a5: F32 router                                                            */
/* ------------------------------------------------------------------------- */

/* tensor.cpp:186-200: bias first, sequential unfused sum over columns. */
void orc_matvec_add_f32(const float *weights, const float *bias, size_t rows, size_t cols,
                        const float *input, float *output) {
    for (size_t row = 0; row < rows; ++row) {
        float sum = bias[row];
        for (size_t column = 0; column < cols; ++column) {
            sum += weights[row * cols + column] * input[column];
        }
        output[row] = sum;
    }
}

/* tensor.cpp:497-527: per (row, token) the same order as the matvec. */
void orc_matmul_add_f32(const float *weights, const float *bias, size_t rows, size_t cols,
                        const float *input, size_t tokens, float *output, float *workspace,
                        float *transposed) {
    for (size_t token = 0; token < tokens; ++token) {
        for (size_t column = 0; column < cols; ++column) {
            transposed[column * tokens + token] = input[token * cols + column];
        }
    }
    for (size_t row = 0; row < rows; ++row) {
        for (size_t token = 0; token < tokens; ++token) {
            workspace[token] = bias[row];
        }
        for (size_t column = 0; column < cols; ++column) {
            const float weight = weights[row * cols + column];
            const float *column_input = transposed + column * tokens;
            for (size_t token = 0; token < tokens; ++token) {
                workspace[token] += weight * column_input[token];
            }
        }
        for (size_t token = 0; token < tokens; ++token) {
            output[token * rows + row] = workspace[token];
        }
    }
}

/* ------------------------------------------------------------------------- */
/* a6: top-k + softmax                                                       */
/* ------------------------------------------------------------------------- */

/* std::max(a, b) is (a < b) ? b : a; std::min(a, b) is (b < a) ? b : a. */
static float std_max(float a, float b) {
    return (a < b) ? b : a;
}

static float std_min(float a, float b) {
    return (b < a) ? b : a;
}

/* model.cpp:296-321: partial selection sort over an index permutation with a
 * strict '>' (so the earliest current position wins a tie, and a NaN already
 * at the current position is never displaced), then a softmax over the k
 * selected logits: max, exp(l - max), sequential sum, divide. */
void orc_router_topk(const float *logits, size_t experts, size_t k, int64_t *indices, float *weights) {
    size_t order[512];
    for (size_t i = 0; i < experts; ++i) {
        order[i] = i;
    }
    for (size_t i = 0; i < k; ++i) {
        size_t best = i;
        for (size_t j = i + 1; j < experts; ++j) {
            if (logits[order[j]] > logits[order[best]]) {
                best = j;
            }
        }
        const size_t tmp = order[i];
        order[i] = order[best];
        order[best] = tmp;
    }
    float maximum = -INFINITY;
    for (size_t i = 0; i < k; ++i) {
        maximum = std_max(maximum, logits[order[i]]);
    }
    float weight_sum = 0.0f;
    for (size_t i = 0; i < k; ++i) {
        weights[i] = expf(logits[order[i]] - maximum);
        weight_sum += weights[i];
    }
    for (size_t i = 0; i < k; ++i) {
        weights[i] /= weight_sum;
        indices[i] = (int64_t)order[i];
    }
}

/* ------------------------------------------------------------------------- */
/* a7: clamped SwiGLU                                                        */
/* ------------------------------------------------------------------------- */

/* model.cpp:328-332: x = min(gate, 7), y = clamp(up, -7, 7),
 * h = (x / (1 + exp(-1.702 x))) * (y + 1). */
void orc_swiglu(const float *gate, const float *up, size_t n, float *hidden) {
    for (size_t i = 0; i < n; ++i) {
        const float x = std_min(gate[i], 7.0f);
        const float u = up[i];
        const float y = (u < -7.0f) ? -7.0f : ((7.0f < u) ? 7.0f : u);
        hidden[i] = (x / (1.0f + expf(-1.702f * x))) * (y + 1.0f);
    }
}

/* ------------------------------------------------------------------------- */
/* a8/a9: MoE                                                                */
/* ------------------------------------------------------------------------- */

#define ORC_MAX_WIDTH 8192

/* model.cpp:292-338 */
void orc_moe(const orc_moe_layer *layer, const float *input, float *output, int body, float *router_out,
             int64_t *indices_out, float *weights_out) {
    float router[512];
    int64_t indices[16];
    float weights[16];
    static float gate[ORC_MAX_WIDTH], up[ORC_MAX_WIDTH], hidden[ORC_MAX_WIDTH], down[ORC_MAX_WIDTH];

    orc_matvec_add_f32(layer->router_weight, layer->router_bias, layer->experts, layer->hidden, input, router);
    orc_router_topk(router, layer->experts, layer->used, indices, weights);

    for (size_t i = 0; i < layer->hidden; ++i) {
        output[i] = 0.0f;
    }
    for (size_t selected = 0; selected < layer->used; ++selected) {
        const size_t expert = (size_t)indices[selected];
        orc_matvec_add_mxfp4(layer->gate_weight, layer->gate_bias, layer->expert_hidden, layer->hidden, input, gate,
                             expert, body);
        orc_matvec_add_mxfp4(layer->up_weight, layer->up_bias, layer->expert_hidden, layer->hidden, input, up,
                             expert, body);
        orc_swiglu(gate, up, layer->expert_hidden, hidden);
        orc_matvec_add_mxfp4(layer->down_weight, layer->down_bias, layer->hidden, layer->expert_hidden, hidden,
                             down, expert, body);
        for (size_t i = 0; i < layer->hidden; ++i) {
            output[i] += weights[selected] * down[i];
        }
    }
    if (router_out) {
        memcpy(router_out, router, layer->experts * sizeof(float));
    }
    if (indices_out) {
        memcpy(indices_out, indices, layer->used * sizeof(int64_t));
    }
    if (weights_out) {
        memcpy(weights_out, weights, layer->used * sizeof(float));
    }
}

/* model.cpp:378-460 with the routing given: buckets per expert in token order,
 * then per expert (ascending index): per-token matvecs when at most 4 tokens
 * chose it (model.cpp:22,404), the selected-token matmul otherwise; SwiGLU; down;
 * out[token] += w * down in expert-index order, from 0. */
void orc_moe_batch_experts(const orc_moe_layer *layer, const float *input, size_t count, const int64_t *indices,
                           const float *weights, float *output, int body) {
    const size_t H = layer->hidden, F = layer->expert_hidden, E = layer->experts, K = layer->used;
    const size_t width = H > F ? H : F;
    float *workspace = malloc(sizeof(float) * count * 4 + sizeof(float) * count);
    float *transposed = malloc(sizeof(float) * count * width);
    size_t *bucket_tokens = malloc(sizeof(size_t) * count * E);
    float *bucket_weights = malloc(sizeof(float) * count * E);
    size_t *bucket_counts = calloc(E, sizeof(size_t));
    float *gate = malloc(sizeof(float) * count * F);
    float *up = malloc(sizeof(float) * count * F);
    float *hidden = malloc(sizeof(float) * count * F);
    float *down = malloc(sizeof(float) * count * H);

    for (size_t i = 0; i < count * H; ++i) {
        output[i] = 0.0f;
    }
    for (size_t p = 0; p < count; ++p) {
        for (size_t r = 0; r < K; ++r) {
            const size_t e = (size_t)indices[p * K + r];
            const size_t offset = e * count + bucket_counts[e];
            bucket_tokens[offset] = p;
            bucket_weights[offset] = weights[p * K + r];
            ++bucket_counts[e];
        }
    }
    for (size_t e = 0; e < E; ++e) {
        const size_t n = bucket_counts[e];
        if (n == 0) {
            continue;
        }
        const size_t *tokens = bucket_tokens + e * count;
        const float *token_weights = bucket_weights + e * count;
        if (n <= 4) {
            for (size_t s = 0; s < n; ++s) {
                const size_t p = tokens[s];
                orc_matvec_add_mxfp4(layer->gate_weight, layer->gate_bias, F, H, input + p * H, gate + p * F, e, body);
                orc_matvec_add_mxfp4(layer->up_weight, layer->up_bias, F, H, input + p * H, up + p * F, e, body);
            }
        } else {
            orc_transpose_selected(H, input, tokens, n, transposed);
            orc_matmul_add_mxfp4_selected_transposed(layer->gate_weight, layer->gate_bias, F, H, transposed, tokens,
                                                     n, gate, workspace, e, body);
            orc_matmul_add_mxfp4_selected_transposed(layer->up_weight, layer->up_bias, F, H, transposed, tokens, n,
                                                     up, workspace, e, body);
        }
        for (size_t s = 0; s < n; ++s) {
            const size_t p = tokens[s];
            orc_swiglu(gate + p * F, up + p * F, F, hidden + p * F);
        }
        if (n <= 4) {
            for (size_t s = 0; s < n; ++s) {
                const size_t p = tokens[s];
                orc_matvec_add_mxfp4(layer->down_weight, layer->down_bias, H, F, hidden + p * F, down + p * H, e,
                                     body);
            }
        } else {
            orc_transpose_selected(F, hidden, tokens, n, transposed);
            orc_matmul_add_mxfp4_selected_transposed(layer->down_weight, layer->down_bias, H, F, transposed, tokens,
                                                     n, down, workspace, e, body);
        }
        for (size_t s = 0; s < n; ++s) {
            const size_t p = tokens[s];
            const float w = token_weights[s];
            for (size_t i = 0; i < H; ++i) {
                output[p * H + i] += w * down[p * H + i];
            }
        }
    }
    free(workspace);
    free(transposed);
    free(bucket_tokens);
    free(bucket_weights);
    free(bucket_counts);
    free(gate);
    free(up);
    free(hidden);
    free(down);
}

/* model.cpp:340-461.  Router via the F32 matmul, per-token top-k (model.cpp:347-377),
 * then the experts as orc_moe_batch_experts. */
void orc_moe_batch(const orc_moe_layer *layer, const float *input, size_t count, float *output, int body) {
    const size_t H = layer->hidden, E = layer->experts, K = layer->used;
    float *router = malloc(sizeof(float) * count * E);
    float *workspace = malloc(sizeof(float) * count * 4 + sizeof(float) * count);
    float *transposed = malloc(sizeof(float) * count * H);
    int64_t *indices = malloc(sizeof(int64_t) * count * K);
    float *weights = malloc(sizeof(float) * count * K);

    orc_matmul_add_f32(layer->router_weight, layer->router_bias, E, H, input, count, router, workspace,
                       transposed);
    for (size_t p = 0; p < count; ++p) {
        orc_router_topk(router + p * E, E, K, indices + p * K, weights + p * K);
    }
    orc_moe_batch_experts(layer, input, count, indices, weights, output, body);
    free(router);
    free(workspace);
    free(transposed);
    free(indices);
    free(weights);
}

/* ------------------------------------------------------------------------- */
/* a10: RoPE and attention with sinks                                        */
/* ------------------------------------------------------------------------- */

#define ORC_HEAD 64
#define ORC_QHEADS 64
#define ORC_KVHEADS 8
#define ORC_WINDOW 128

/* model.cpp:124-139 with model.h:38,46-50: YaRN frequencies, head 64, base
 * 150000, factor 32, original context 4096, beta_fast 32, beta_slow 1. */
void orc_rope_frequencies(float *frequencies) {
    const float head = 64.0f, base = 150000.0f, scale = 1.0f / 32.0f, original = 4096.0f;
    const float beta_fast = 32.0f, beta_slow = 1.0f;
    const float pi = 3.14159265358979323846f;
    const float corr = head * logf(original / (beta_fast * 2.0f * pi)) / (2.0f * logf(base));
    const float corr_slow = head * logf(original / (beta_slow * 2.0f * pi)) / (2.0f * logf(base));
    const float low = std_max(0.0f, floorf(corr));
    const float high = std_min(head - 1.0f, ceilf(corr_slow));
    for (size_t pair = 0; pair < ORC_HEAD / 2; ++pair) {
        const size_t dimension = pair * 2;
        const float theta_extrap = powf(base, -(float)dimension / head);
        const float y = ((float)pair - low) / std_max(0.001f, high - low);
        const float clamped = (y < 0.0f) ? 0.0f : ((1.0f < y) ? 1.0f : y);
        const float ramp = 1.0f - clamped;
        frequencies[pair] = scale * theta_extrap * (1.0f - ramp) + theta_extrap * ramp;
    }
}

/* model.cpp:230-245: rotate pairs (d, d+32), magnitude 1 + 0.1 ln 32. */
void orc_apply_rope(float *vector, size_t heads, size_t position, const float *frequencies) {
    const float magnitude = 1.0f + 0.1f * logf(1.0f / (1.0f / 32.0f));
    for (size_t head = 0; head < heads; ++head) {
        float *values = vector + head * ORC_HEAD;
        for (size_t pair = 0; pair < ORC_HEAD / 2; ++pair) {
            const float theta = (float)position * frequencies[pair];
            const float cosine = cosf(theta) * magnitude;
            const float sine = sinf(theta) * magnitude;
            const float x = values[pair];
            const float yv = values[pair + ORC_HEAD / 2];
            values[pair] = x * cosine - yv * sine;
            values[pair + ORC_HEAD / 2] = x * sine + yv * cosine;
        }
    }
}

/* model.cpp:36-42 */
static float dot_sequential(const float *a, const float *b, size_t n) {
    float result = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        result += a[i] * b[i];
    }
    return result;
}

/* model.cpp:255-290: even layers see the last 128 positions, odd layers all;
 * query head h reads kv head h/8; the sink joins the max and the denominator
 * but contributes no value. */
void orc_attention(const float *query, const float *key_cache, const float *value_cache, const float *sinks,
                   size_t layer_index, size_t position, float *output, float *scores) {
    const size_t first = (layer_index % 2 == 0 && position + 1 > ORC_WINDOW) ? position + 1 - ORC_WINDOW : 0;
    const size_t count = position + 1 - first;
    const float scale = 1.0f / sqrtf((float)ORC_HEAD);
    for (size_t head = 0; head < ORC_QHEADS; ++head) {
        const size_t kv_head = head / (ORC_QHEADS / ORC_KVHEADS);
        const float *q = query + head * ORC_HEAD;
        float maximum = sinks[head];
        for (size_t i = 0; i < count; ++i) {
            const float *k = key_cache + ((first + i) * ORC_KVHEADS + kv_head) * ORC_HEAD;
            scores[i] = dot_sequential(q, k, ORC_HEAD) * scale;
            maximum = std_max(maximum, scores[i]);
        }
        float denominator = expf(sinks[head] - maximum);
        for (size_t i = 0; i < count; ++i) {
            scores[i] = expf(scores[i] - maximum);
            denominator += scores[i];
        }
        float *result = output + head * ORC_HEAD;
        for (size_t d = 0; d < ORC_HEAD; ++d) {
            result[d] = 0.0f;
        }
        for (size_t i = 0; i < count; ++i) {
            const float weight = scores[i] / denominator;
            const float *v = value_cache + ((first + i) * ORC_KVHEADS + kv_head) * ORC_HEAD;
            for (size_t d = 0; d < ORC_HEAD; ++d) {
                result[d] += weight * v[d];
            }
        }
    }
}

/* ------------------------------------------------------------------------- */
/* a11: RMSNorm                                                              */
/* ------------------------------------------------------------------------- */

/* tensor.cpp:568-580 */
void orc_rms_norm(const float *input, const float *weight, size_t n, float epsilon, float *output) {
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        sum += input[i] * input[i];
    }
    const float scale = 1.0f / sqrtf(sum / (float)n + epsilon);
    for (size_t i = 0; i < n; ++i) {
        output[i] = input[i] * scale * weight[i];
    }
}

/* ------------------------------------------------------------------------- */
/* a12: Q8_0                                                                 */
/* ------------------------------------------------------------------------- */

static uint16_t load_u16(const uint8_t *p) {
    uint16_t v;
    memcpy(&v, p, 2);
    return v;
}

/* tensor.cpp:171-184 */
void orc_load_token_embedding_q8_0(const uint8_t *data, size_t cols, size_t row, float *output) {
    const size_t row_bytes = cols / 32 * 34;
    const uint8_t *base = data + row * row_bytes;
    for (size_t block = 0; block < cols / 32; ++block) {
        const uint8_t *source = base + block * 34;
        const float scale = orc_fp16_to_fp32(load_u16(source));
        const int8_t *quants = (const int8_t *)(source + 2);
        for (size_t i = 0; i < 32; ++i) {
            output[block * 32 + i] = scale * (float)quants[i];
        }
    }
}

/* tensor.cpp:94-114,202-218: two 16-lane accumulators, lane i gets
 * (q_i * d) * x_i for the first and second halves of each block (each
 * product rounded, then added), then lanes are summed pairwise acc0+acc1 and
 * reduced sequentially from 0. */
static float q8_0_row(const uint8_t *data, size_t cols, const float *input) {
    float acc0[16] = {0}, acc1[16] = {0}, acc[16];
    for (size_t block = 0; block < cols / 32; ++block) {
        const uint8_t *source = data + block * 34;
        const float scale = orc_fp16_to_fp32(load_u16(source));
        const int8_t *q = (const int8_t *)(source + 2);
        const float *x = input + block * 32;
        for (size_t i = 0; i < 16; ++i) {
            const float q0 = (float)q[i] * scale;
            const float q1 = (float)q[16 + i] * scale;
            acc0[i] += q0 * x[i];
            acc1[i] += q1 * x[16 + i];
        }
    }
    for (size_t i = 0; i < 16; ++i) {
        acc[i] = acc0[i] + acc1[i];
    }
    return reduce_sequential16(acc);
}

void orc_matvec_q8_0(const uint8_t *data, size_t rows, size_t cols, const float *input, float *output) {
    const size_t row_bytes = cols / 32 * 34;
    for (size_t row = 0; row < rows; ++row) {
        output[row] = q8_0_row(data + row * row_bytes, cols, input);
    }
}

/* tensor.cpp:220-237 */
void orc_matvec_add_q8_0(const uint8_t *data, const float *bias, size_t rows, size_t cols, const float *input,
                         float *output) {
    const size_t row_bytes = cols / 32 * 34;
    for (size_t row = 0; row < rows; ++row) {
        output[row] = bias[row] + q8_0_row(data + row * row_bytes, cols, input);
    }
}

/* tensor.cpp:529-566: per (row, token) bias first, then sequential unfused
 * (d*q) * x over the columns -- a different order from the matvec. */
void orc_matmul_add_q8_0(const uint8_t *data, const float *bias, size_t rows, size_t cols, const float *input,
                         size_t tokens, float *output, float *workspace, float *transposed) {
    const size_t row_bytes = cols / 32 * 34;
    for (size_t token = 0; token < tokens; ++token) {
        for (size_t column = 0; column < cols; ++column) {
            transposed[column * tokens + token] = input[token * cols + column];
        }
    }
    for (size_t row = 0; row < rows; ++row) {
        const uint8_t *base = data + row * row_bytes;
        for (size_t token = 0; token < tokens; ++token) {
            workspace[token] = bias[row];
        }
        for (size_t block = 0; block < cols / 32; ++block) {
            const uint8_t *source = base + block * 34;
            const float scale = orc_fp16_to_fp32(load_u16(source));
            const int8_t *quants = (const int8_t *)(source + 2);
            for (size_t i = 0; i < 32; ++i) {
                const float weight = scale * (float)quants[i];
                const float *column_input = transposed + (block * 32 + i) * tokens;
                for (size_t token = 0; token < tokens; ++token) {
                    workspace[token] += weight * column_input[token];
                }
            }
        }
        for (size_t token = 0; token < tokens; ++token) {
            output[token * rows + row] = workspace[token];
        }
    }
}

void orc_matvec_bf16(const uint16_t *weights, size_t rows, size_t cols, const float *input, float *output) {
    for (size_t row = 0; row < rows; ++row) {
        float sum = 0.0f;
        for (size_t column = 0; column < cols; ++column) {
            sum += orc_bf16_to_fp32(weights[row * cols + column]) * input[column];
        }
        output[row] = sum;
    }
}

/* ------------------------------------------------------------------------- */
/* a13: greedy                                                               */
/* ------------------------------------------------------------------------- */

/* model.cpp:604-612: first index whose logit is strictly greater than every
 * earlier one; a NaN at index 0 is never displaced. */
int32_t orc_greedy(const float *logits, size_t n) {
    size_t best = 0;
    for (size_t i = 1; i < n; ++i) {
        if (logits[i] > logits[best]) {
            best = i;
        }
    }
    return (int32_t)best;
}

/* ------------------------------------------------------------------------- */
/* one transformer block                                                     */
/* ------------------------------------------------------------------------- */

/* model.cpp:572-595 (with model.h:34-44 widths) */
void orc_layer_forward(const orc_layer *layer, size_t layer_index, size_t position, const float *x_in,
                       const float *rope_frequencies, float *key_cache, float *value_cache, int body, float *x_out,
                       float *query_out, float *attended_out, float *residual_out, float *router_out,
                       int64_t *indices_out, float *weights_out) {
    enum { H = 2880, QW = ORC_QHEADS * ORC_HEAD, KW = ORC_KVHEADS * ORC_HEAD };
    static float normalized[H], query[QW], key[KW], value[KW], attended[QW], projected[H], residual[H],
        moe_out[H];
    float *scores = malloc(sizeof(float) * (position + 1));
    orc_rms_norm(x_in, layer->attention_norm, H, 1.0e-5f, normalized);
    orc_matvec_add_q8_0(layer->query_weight, layer->query_bias, QW, H, normalized, query);
    orc_matvec_add_q8_0(layer->key_weight, layer->key_bias, KW, H, normalized, key);
    orc_matvec_add_q8_0(layer->value_weight, layer->value_bias, KW, H, normalized, value);
    orc_apply_rope(query, ORC_QHEADS, position, rope_frequencies);
    orc_apply_rope(key, ORC_KVHEADS, position, rope_frequencies);
    memcpy(key_cache + position * KW, key, sizeof(key));     /* store_kv, model.cpp:247-253 */
    memcpy(value_cache + position * KW, value, sizeof(value));
    orc_attention(query, key_cache, value_cache, layer->sinks, layer_index, position, attended, scores);
    orc_matvec_add_q8_0(layer->output_weight, layer->output_bias, H, QW, attended, projected);
    for (size_t j = 0; j < H; ++j) {
        residual[j] = x_in[j] + projected[j];
    }
    orc_rms_norm(residual, layer->post_attention_norm, H, 1.0e-5f, normalized);
    orc_moe(&layer->moe, normalized, moe_out, body, router_out, indices_out, weights_out);
    for (size_t j = 0; j < H; ++j) {
        x_out[j] = residual[j] + moe_out[j];
    }
    if (query_out) {
        memcpy(query_out, query, sizeof(query));
    }
    if (attended_out) {
        memcpy(attended_out, attended, sizeof(attended));
    }
    if (residual_out) {
        memcpy(residual_out, residual, sizeof(residual));
    }
    free(scores);
}

/* model.cpp:484-553 for positions first .. first + count - 1. */
void orc_layer_prefill(const orc_layer *layer, size_t layer_index, size_t first, size_t count, const float *x_in,
                       const float *rope_frequencies, float *key_cache, float *value_cache, int body, float *x_out,
                       float *residual_out) {
    enum { H = 2880, QW = ORC_QHEADS * ORC_HEAD, KW = ORC_KVHEADS * ORC_HEAD };
    if (count == 0) {
        return;
    }
    float *normalized = calloc(count * H, sizeof(float));
    float *query = malloc(sizeof(float) * count * QW);
    float *key = malloc(sizeof(float) * count * KW);
    float *value = malloc(sizeof(float) * count * KW);
    float *attended = malloc(sizeof(float) * count * QW);
    float *projected = malloc(sizeof(float) * count * H);
    float *residual = malloc(sizeof(float) * count * H);
    float *moe_out = malloc(sizeof(float) * count * H);
    float *workspace = malloc(sizeof(float) * count);
    float *transposed = malloc(sizeof(float) * count * QW);
    float *scores = malloc(sizeof(float) * (first + count));

    for (size_t p = 0; p < count; ++p) {
        orc_rms_norm(x_in + p * H, layer->attention_norm, H, 1.0e-5f, normalized + p * H);
    }
    orc_matmul_add_q8_0(layer->query_weight, layer->query_bias, QW, H, normalized, count, query, workspace,
                        transposed);
    orc_matmul_add_q8_0(layer->key_weight, layer->key_bias, KW, H, normalized, count, key, workspace, transposed);
    orc_matmul_add_q8_0(layer->value_weight, layer->value_bias, KW, H, normalized, count, value, workspace,
                        transposed);
    for (size_t p = 0; p < count; ++p) {
        orc_apply_rope(query + p * QW, ORC_QHEADS, first + p, rope_frequencies);
        orc_apply_rope(key + p * KW, ORC_KVHEADS, first + p, rope_frequencies);
        memcpy(key_cache + (first + p) * KW, key + p * KW, sizeof(float) * KW); /* store_kv */
        memcpy(value_cache + (first + p) * KW, value + p * KW, sizeof(float) * KW);
    }
    for (size_t p = 0; p < count; ++p) {
        orc_attention(query + p * QW, key_cache, value_cache, layer->sinks, layer_index, first + p, attended + p * QW,
                      scores);
    }
    orc_matmul_add_q8_0(layer->output_weight, layer->output_bias, H, QW, attended, count, projected, workspace,
                        transposed);
    for (size_t p = 0; p < count; ++p) {
        for (size_t j = 0; j < H; ++j) {
            residual[p * H + j] = x_in[p * H + j] + projected[p * H + j];
        }
        orc_rms_norm(residual + p * H, layer->post_attention_norm, H, 1.0e-5f, normalized + p * H);
    }
    orc_moe_batch(&layer->moe, normalized, count, moe_out, body);
    for (size_t p = 0; p < count; ++p) {
        for (size_t j = 0; j < H; ++j) {
            x_out[p * H + j] = residual[p * H + j] + moe_out[p * H + j];
        }
    }
    if (residual_out) {
        memcpy(residual_out, residual, sizeof(float) * count * H);
    }
    free(normalized);
    free(query);
    free(key);
    free(value);
    free(attended);
    free(projected);
    free(residual);
    free(moe_out);
    free(workspace);
    free(transposed);
    free(scores);
}

/* ------------------------------------------------------------------------- */
/* synthetic inputs                                                          */
/* ------------------------------------------------------------------------- */

/* splitmix64 finaliser applied to a Weyl sequence: element `index` of stream
 * `stream` is independent of every other, so any slice can be regenerated. */
static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t orc_hash(uint64_t seed, uint64_t stream, uint64_t index) {
    return mix64(seed + stream * 0xD1342543DE82EF95ull + (index + 1) * 0x9E3779B97F4A7C15ull);
}

static float synth_unit_normal(uint64_t seed, uint64_t stream, uint64_t i) {
    int32_t sum = 0;
    for (uint64_t j = 0; j < 12; ++j) {
        sum += (int32_t)(orc_hash(seed, stream, 12 * i + j) >> 40);
    }
    sum -= 6 << 24;
    return (float)sum * 0x1p-24f;
}

void orc_synth_normal(uint64_t seed, uint64_t stream, size_t offset, size_t n, float mean, float sigma,
                      float *out) {
    for (size_t i = 0; i < n; ++i) {
        out[i] = mean + synth_unit_normal(seed, stream, offset + i) * sigma;
    }
}

void orc_synth_normal_bf16(uint64_t seed, uint64_t stream, size_t offset, size_t n, float sigma, float *out) {
    for (size_t i = 0; i < n; ++i) {
        out[i] = orc_bf16_to_fp32(orc_fp32_to_bf16(synth_unit_normal(seed, stream, offset + i) * sigma));
    }
}

void orc_synth_mxfp4(uint64_t seed, uint64_t stream, size_t block_offset, size_t n, uint32_t emin,
                     uint32_t emax, uint8_t *out) {
    const uint64_t span = (uint64_t)(emax - emin + 1);
    for (size_t k = 0; k < n; ++k) {
        const uint64_t b = block_offset + k;
        uint8_t *block = out + k * 17;
        block[0] = (uint8_t)(emin + orc_hash(seed, stream, 3 * b) % span);
        const uint64_t lo = orc_hash(seed, stream, 3 * b + 1);
        const uint64_t hi = orc_hash(seed, stream, 3 * b + 2);
        for (int i = 0; i < 8; ++i) {
            block[1 + i] = (uint8_t)(lo >> (8 * i));
            block[9 + i] = (uint8_t)(hi >> (8 * i));
        }
    }
}

void orc_synth_q8_0(uint64_t seed, uint64_t stream, size_t block_offset, size_t n, uint8_t *out) {
    for (size_t k = 0; k < n; ++k) {
        const uint64_t b = block_offset + k;
        uint8_t *block = out + k * 34;
        const uint16_t scale = (uint16_t)(0x0c00u | (orc_hash(seed, stream, 5 * b) & 0x3ffu));
        memcpy(block, &scale, 2);
        for (int w = 0; w < 4; ++w) {
            const uint64_t h = orc_hash(seed, stream, 5 * b + 1 + (uint64_t)w);
            for (int i = 0; i < 8; ++i) {
                block[2 + 8 * w + i] = (uint8_t)(h >> (8 * i));
            }
        }
    }
}

void orc_synth_bf16(uint64_t seed, uint64_t stream, size_t offset, size_t n, uint16_t *out) {
    for (size_t k = 0; k < n; ++k) {
        const uint64_t i = offset + k;
        const uint32_t h = (uint32_t)(orc_hash(seed, stream, i >> 2) >> (16 * (i & 3))) & 0xffffu;
        out[k] = (uint16_t)((h & 0x807fu) | ((120u + ((h >> 7) & 3u)) << 7));
    }
}
