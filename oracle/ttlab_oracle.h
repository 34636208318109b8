/*
 * ttlab_oracle.h -- CPU restatement of tt-lab's quantized decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (tt-lab_amd/) links, loads or
 * calls this library.  Only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py use it, and only as the checker or as the timed CPU baseline.
 *
 * Every function restates one function of the reference C++ implementation
 * (tenstorrent/tt-lab, src/tensor.cpp and src/model.cpp) in plain C11, keeping the
 * reference's operation order and rounding points.  The library is compiled with
 * -O3 -ffp-contract=off -march=x86-64-v3, the reference's own flags (rules.py:6-11),
 * so the "default" bodies never fuse a multiply and an add.  The reference's
 * AVX-512 ("v4") bodies are restated twice: lane by lane in portable C with fmaf
 * (ORC_BODY_V4, runs on any x86-64-v3 host) and with AVX-512 intrinsics
 * (ORC_BODY_V4_SIMD, used for CPU-baseline timing; requires avx512f+bw).
 *
 * Pinning (each function is checked by tests/test_oracle_*.py against):
 *   - the reference's own known-answer tests: src/tests.cpp:38-52,194-234 and
 *     tests/host_dispatch.cpp:92-127 (1080.25 MXFP4 KAT, selected-matmul KAT);
 *   - closed forms (exhaustive 16 codes x 256 E8M0 scales against ldexp);
 *   - brute-force double-precision dot products on small and 2880-wide shapes;
 *   - cross-body agreement (default vs v4 vs v4-simd) and exact v4 == v4-simd;
 *   - for the MoE routing (model.cpp:296-321): brute-force full sorts with the
 *     tie/NaN rules of the selection sort.
 * Functions with no reference test and no closed form that fixes them exactly
 * (SwiGLU, attention softmax, RoPE, full-layer composition) are pinned only by
 * brute force in double within tolerance; their headers below say
 * "parity unpinned" for the bit level.
 *
 * The synthetic-input generators at the end are the shared specification that
 * the device generators in tt-lab_amd/csrc/ttl_synth.hip also implement; the tests
 * compare the two bit for bit.
 */
#ifndef TTLAB_ORACLE_H
#define TTLAB_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Body selectors for the functions the reference multiversions (tensor.h:28-51). */
#define ORC_BODY_DEFAULT 0  /* [[gnu::target("default")]] bodies: scalar, unfused   */
#define ORC_BODY_V4 1       /* arch=x86-64-v4 bodies restated lane by lane with fmaf */
#define ORC_BODY_V4_SIMD 2  /* arch=x86-64-v4 bodies with AVX-512 intrinsics         */

/* GGUF tensor type ids (tensor.h:11-13) plus BF16 (GGML type 30). */
#define ORC_TYPE_F32 0u
#define ORC_TYPE_Q8_0 8u
#define ORC_TYPE_BF16 30u
#define ORC_TYPE_MXFP4 39u

int orc_has_avx512(void);

/* ---- a1: formats ------------------------------------------------------- */
float orc_mxfp4_scale(uint8_t exponent);            /* tensor.cpp:36-44,167-169   */
int orc_mxfp4_int(uint8_t code);                    /* tensor.cpp:34              */
float orc_fp16_to_fp32(uint16_t half);              /* tensor.cpp:163-165         */
uint16_t orc_fp32_to_bf16(float value);             /* requant.cpp:311-316        */
float orc_bf16_to_fp32(uint16_t bits);
/* Decodes n GGUF MXFP4 blocks (17 B each) into 32*n floats, element order as
 * tensor.cpp:283-296: byte 1+i low nibble -> element i, high nibble -> i+16. */
void orc_mxfp4_dequant_blocks(const uint8_t *blocks, size_t n, float *out);

/* ---- a2: layout ---------------------------------------------------------- */
int64_t orc_tensor_row_bytes(uint32_t type, uint64_t n); /* tensor.cpp:136-157; -1 on error */

/* ---- a3: MXFP4 matvec (tensor.cpp:239-304) -------------------------------
 * y[r] = bias[expert][r] + sum_k W[expert][r][k] x[k].  The reference fixes
 * rows = cols = 2880; the restatement takes both (cols % 32 == 0, and for the
 * default body rows % 4 == 0 as its 4-row interleave requires).            */
void orc_matvec_add_mxfp4(const uint8_t *matrix, const float *bias, size_t rows, size_t cols,
                          const float *input, float *output, size_t expert, int body);

/* ---- a4: selected-token MXFP4 matmul (tensor.cpp:306-495) ---------------- */
void orc_transpose_selected(size_t cols, const float *input, const size_t *tokens, size_t count,
                            float *transposed);
void orc_matmul_add_mxfp4_selected_transposed(const uint8_t *matrix, const float *bias, size_t rows,
                                              size_t cols, const float *transposed, const size_t *tokens,
                                              size_t count, float *output, float *workspace, size_t expert,
                                              int body);

/* ---- a5: F32 router matvec / matmul (tensor.cpp:186-200,497-527) -------- */
void orc_matvec_add_f32(const float *weights, const float *bias, size_t rows, size_t cols,
                        const float *input, float *output);
void orc_matmul_add_f32(const float *weights, const float *bias, size_t rows, size_t cols,
                        const float *input, size_t tokens, float *output, float *workspace,
                        float *transposed);

/* ---- a6: top-k selection + softmax (model.cpp:296-321) ------------------- */
void orc_router_topk(const float *logits, size_t experts, size_t k, int64_t *indices, float *weights);

/* ---- a7: clamped SwiGLU (model.cpp:328-332), parity unpinned at the bit level (libm expf) */
void orc_swiglu(const float *gate, const float *up, size_t n, float *hidden);

/* ---- a8/a9: one decode MoE layer (model.cpp:292-338) --------------------- */
typedef struct {
    size_t hidden;          /* embedding length, 2880            */
    size_t expert_hidden;   /* expert feed-forward length, 2880  */
    size_t experts;         /* 32 (20b) or 128 (120b)            */
    size_t used;            /* experts per token, 4              */
    const float *router_weight;  /* f32 [experts][hidden]       */
    const float *router_bias;    /* f32 [experts]               */
    const uint8_t *gate_weight;  /* MXFP4 [experts][expert_hidden][hidden/32][17] */
    const float *gate_bias;      /* f32 [experts][expert_hidden] */
    const uint8_t *up_weight;
    const float *up_bias;
    const uint8_t *down_weight;  /* MXFP4 [experts][hidden][expert_hidden/32][17] */
    const float *down_bias;      /* f32 [experts][hidden]        */
} orc_moe_layer;

/* Writes out[hidden]; optionally router logits[experts], indices[used], weights[used]. */
void orc_moe(const orc_moe_layer *layer, const float *input, float *output, int body, float *router_out,
             int64_t *indices_out, float *weights_out);

/* model.cpp:340-461: prefill MoE over `count` tokens (layer-major, expert-order combine). */
void orc_moe_batch(const orc_moe_layer *layer, const float *input, size_t count, float *output, int body);
/* model.cpp:378-460, the experts of orc_moe_batch with the routing given: indices
 * int64 [count][used] (each in 0..experts-1), weights f32 [count][used]. */
void orc_moe_batch_experts(const orc_moe_layer *layer, const float *input, size_t count, const int64_t *indices,
                           const float *weights, float *output, int body);

/* ---- a10: RoPE and attention with sinks (model.cpp:124-139,230-290) ------ */
void orc_rope_frequencies(float *frequencies /* [32] */);
void orc_apply_rope(float *vector, size_t heads, size_t position, const float *frequencies);
/* kv caches: f32 [positions][8][64]; query f32 [64][64]; output f32 [64][64]; scores scratch [position+1]. */
void orc_attention(const float *query, const float *key_cache, const float *value_cache, const float *sinks,
                   size_t layer_index, size_t position, float *output, float *scores);

/* ---- a11: RMSNorm (tensor.cpp:568-580) ----------------------------------- */
void orc_rms_norm(const float *input, const float *weight, size_t n, float epsilon, float *output);

/* ---- a12: Q8_0 (tensor.cpp:94-114,171-237,529-566) ----------------------- */
void orc_load_token_embedding_q8_0(const uint8_t *data, size_t cols, size_t row, float *output);
void orc_matvec_q8_0(const uint8_t *data, size_t rows, size_t cols, const float *input, float *output);
void orc_matvec_add_q8_0(const uint8_t *data, const float *bias, size_t rows, size_t cols, const float *input,
                         float *output);
void orc_matmul_add_q8_0(const uint8_t *data, const float *bias, size_t rows, size_t cols, const float *input,
                         size_t tokens, float *output, float *workspace, float *transposed);

/* BF16 unembedding for the synthetic 20b/120b configurations.  The reference's
 * output.weight is Q8_0; it has no BF16 matvec.  This is the reference's F32
 * matvec order (tensor.cpp:186-200, no bias) over BF16 weights widened exactly
 * to f32.  No reference counterpart: parity unpinned against the reference,
 * pinned against brute force. */
void orc_matvec_bf16(const uint16_t *weights, size_t rows, size_t cols, const float *input, float *output);

/* ---- a13: greedy (model.cpp:604-612) -------------------------------------- */
int32_t orc_greedy(const float *logits, size_t n);

/* One gpt-oss transformer block's tensors (GGUF layouts; names as model.cpp:141-169). */
typedef struct {
    const float *attention_norm;     /* f32 [2880] */
    const float *post_attention_norm;
    const uint8_t *query_weight;     /* Q8_0 4096 x 2880 */
    const float *query_bias;         /* f32 [4096] */
    const uint8_t *key_weight;       /* Q8_0 512 x 2880 */
    const float *key_bias;
    const uint8_t *value_weight;     /* Q8_0 512 x 2880 */
    const float *value_bias;
    const uint8_t *output_weight;    /* Q8_0 2880 x 4096 */
    const float *output_bias;        /* f32 [2880] */
    const float *sinks;              /* f32 [64] */
    orc_moe_layer moe;
} orc_layer;

/* The body of GptOssModel::forward's layer loop (model.cpp:571-595) for one layer
 * at `position`: writes key/value for `position` into the caches (f32
 * [capacity][8][64]), reads positions before it, and writes the layer output
 * x_out[2880].  Optional outputs (each may be NULL): query[4096] after RoPE,
 * attended[4096], residual[2880], router[experts], indices[used], weights[used]. */
void orc_layer_forward(const orc_layer *layer, size_t layer_index, size_t position, const float *x_in,
                       const float *rope_frequencies, float *key_cache, float *value_cache, int body, float *x_out,
                       float *query, float *attended, float *residual, float *router, int64_t *indices,
                       float *weights);

/* The body of GptOssModel::prefill's layer loop (model.cpp:484-553) for `count`
 * tokens at positions first .. first+count-1 (the reference's prefill has first = 0):
 * per-token RMSNorm, the batched Q8_0 matmuls (matmul_add_q8_0), RoPE and the KV
 * store of every token, then attention per token, the output matmul, the residual,
 * moe_batch and the second residual.  x_in/x_out f32 [count][2880]; the caches as in
 * orc_layer_forward.  residual_out [count][2880] may be NULL.  Pinned against an
 * independent float64 restatement of the same layer body (tests/brute_force.py,
 * layer_prefill), with mutation checks on the norms and the attention window. */
void orc_layer_prefill(const orc_layer *layer, size_t layer_index, size_t first, size_t count, const float *x_in,
                       const float *rope_frequencies, float *key_cache, float *value_cache, int body, float *x_out,
                       float *residual_out);

/* ---- synthetic inputs (shared specification with tt-lab_amd/csrc/ttl_synth.hip) */
uint64_t orc_hash(uint64_t seed, uint64_t stream, uint64_t index);
/* N(0,1) drawn as an Irwin-Hall sum of 12 24-bit uniforms in exact integer arithmetic,
 * times sigma, plus mean. */
void orc_synth_normal(uint64_t seed, uint64_t stream, size_t offset, size_t n, float mean, float sigma,
                      float *out);
/* Same values rounded to BF16 (requant.cpp:311-316) and widened back to f32. */
void orc_synth_normal_bf16(uint64_t seed, uint64_t stream, size_t offset, size_t n, float sigma, float *out);
/* GGUF MXFP4 blocks: E8M0 uniform in [emin, emax], 32 nibble codes uniform over 16. */
void orc_synth_mxfp4(uint64_t seed, uint64_t stream, size_t block_offset, size_t n, uint32_t emin,
                     uint32_t emax, uint8_t *out);
/* GGUF Q8_0 blocks: fp16 scale in [2^-12, 2^-11), int8 quants uniform. */
void orc_synth_q8_0(uint64_t seed, uint64_t stream, size_t block_offset, size_t n, uint8_t *out);
/* BF16 bits: random sign and mantissa, exponent uniform in 120..123. */
void orc_synth_bf16(uint64_t seed, uint64_t stream, size_t offset, size_t n, uint16_t *out);

#ifdef __cplusplus
}
#endif

#endif
