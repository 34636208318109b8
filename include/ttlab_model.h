/*
 * ttlab_model.h -- C API of the C++ gpt-oss decode model that runs on the gfx950
 * backend (tt-lab_amd/host/gpt_oss_hip.{hpp,cpp}, class ttlab::HipGptOssModel).
 *
 * The model mirrors the reference's GptOssModel (model.h:15-31): construction
 * allocates everything, forward(token, position) advances one token and returns
 * logits, greedy() picks the first maximum.  Weights come from a gpt-oss GGUF
 * file (ttlm_create_from_gguf) or are synthetic (the benchmark configurations 3 and
 * 4), generated on the device from the stream layout of ttlab::synth_stream().
 * Every call returns 0 or a negative code; ttlm_last_error() has the message.
 */
#ifndef TTLAB_MODEL_H
#define TTLAB_MODEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ttlm_model ttlm_model;

/* layers >= 1, experts 32 or 128, vocab >= 1, capacity = KV positions (token capacity). */
int ttlm_create_synthetic(int device, uint32_t layers, uint32_t experts, uint32_t vocab, uint32_t capacity,
                          uint64_t seed, ttlm_model **out);
/* A gpt-oss GGUF file (version 3, as the reference's GgufFile reads it, gguf.cpp:145-239):
 * the metadata and tensors GptOssModel's constructor checks (model.cpp:64-206), with
 * its error messages.  strict != 0 applies the reference's limits exactly (24 or 36
 * layers, 32 or 128 experts, vocabulary 201088, Q8_0 output.weight); strict == 0
 * also accepts 1..36 layers, 4..128 experts, a vocabulary that is a multiple of 16
 * and a BF16 output.weight (small test models, bf16-unembedding configurations). */
typedef struct {
    uint32_t layers, experts, vocab;
    uint32_t output_type; /* GGML type of output.weight: 8 (Q8_0) or 30 (BF16) */
    uint32_t tensors;
} ttlm_gguf_info;
/* Checks a file without a device. */
int ttlm_gguf_inspect(const char *path, int strict, ttlm_gguf_info *info);
/* The model with a GGUF file's weights (uploaded to the device, MXFP4 and Q8_0
 * repacked there); capacity = token capacity of the KV caches (model.cpp:64). */
int ttlm_create_from_gguf(const char *path, int device, uint32_t capacity, int strict, ttlm_model **out);
void ttlm_destroy(ttlm_model *model);
const char *ttlm_last_error(void);

/* GptOssModel::forward (model.cpp:557-602): logits (host, f32 [vocab]) may be NULL. */
int ttlm_forward(ttlm_model *model, int32_t token, uint32_t position, float *logits);
/* GptOssModel::prefill (model.cpp:463-555), layer-major on the device: per layer the
 * batched Q8_0 matmuls (MFMA), RoPE and the KV store of every token, attention per
 * token, and moe_batch (MFMA expert GEMMs); logits (host, f32 [vocab], may be NULL) of
 * the last token.  Prompts longer than ttlm_prefill_batch() run in consecutive passes
 * (a token's results do not depend on the cut).  Positions 0 .. count-1 are filled. */
int ttlm_prefill(ttlm_model *model, const int32_t *tokens, uint32_t count, float *logits);
/* Tokens per layer-major prefill pass. */
uint32_t ttlm_prefill_batch(const ttlm_model *model);
/* After a prefill: the inputs of `layer` (layer == layers: the final stream) of the
 * last pass's first `count` tokens, f32 [count][2880] (host). */
int ttlm_prefill_state(ttlm_model *model, uint32_t layer, uint32_t count, float *x_in);
/* Greedy decode on the device: feeds token at position, then each step's argmax,
 * for `steps` steps; tokens (host, int32 [steps]) receives the chosen tokens. */
int ttlm_generate(ttlm_model *model, int32_t token, uint32_t position, uint32_t steps, int32_t *tokens);
/* Times `steps` device-resident decode steps (after `warmup` untimed ones) with HIP
 * events around the graph replays; positions start at `position`. */
int ttlm_time_decode(ttlm_model *model, int32_t token, uint32_t position, uint32_t warmup, uint32_t steps,
                     double *ms_per_step);

/* Microseconds per launch of the MXFP4 gate/up + SwiGLU kernel: every layer's launch
 * with the last step's routing, as one graph replayed `reps` times (HIP events). */
int ttlm_time_expert_kernel(ttlm_model *model, uint32_t reps, double *us_per_launch);

/* The decode step's kernels timed one kind at a time: every launch of `kind` that a step
 * at `position` makes (all layers; the attention kinds only the layers of their parity;
 * logits one), with the last step's inputs and scratch outputs, captured as one graph
 * replayed `reps` times between HIP events.  us_per_launch: microseconds per launch
 * (per partials + combine pair for TTLM_KERNEL_ATTENTION_FULL); launches (may be NULL):
 * launches per replay.  The model's state is unchanged. */
#define TTLM_KERNEL_QKV 0u               /* combine + residual + norm staged, Q8_0 QKV + bias +
                                          * RoPE + KV store (qkv_kernel)                         */
#define TTLM_KERNEL_ATTENTION_WINDOW 1u  /* even layers: attn_window_kernel                     */
#define TTLM_KERNEL_ATTENTION_FULL 2u    /* odd layers: attn_partial_kernel + attn_combine_kernel */
#define TTLM_KERNEL_OUTPUT 3u            /* O projection + residual (q8_matvec_kernel<4096>)     */
#define TTLM_KERNEL_ROUTER_ROWS 4u       /* exact router rows and bounds (router_rows_kernel)    */
#define TTLM_KERNEL_GATEUP_ROUTED 5u     /* gateup_swiglu_kernel with the top-k ranking, as run  */
#define TTLM_KERNEL_GATEUP_GIVEN 6u      /* the same with the indices given                      */
#define TTLM_KERNEL_DOWN 7u              /* the 4 experts' down projections + bias (down_kernel) */
#define TTLM_KERNEL_LOGITS 8u            /* unembedding + per-workgroup argmax                   */
#define TTLM_KERNEL_GATEUP_DOWN 9u       /* gate/up and down in one launch (gateup_down_kernel; the
                                          * step runs them as two, which is faster)               */
int ttlm_time_kernel(ttlm_model *model, uint32_t kind, uint32_t position, uint32_t reps, double *us_per_launch,
                     uint32_t *launches);

/* Decode steps (and the expert-kernel timer) replay captured HIP graphs when `enabled`
 * is nonzero (the default), else launch the same kernels one by one on the model's
 * stream -- for tools that cannot follow graph launches. */
int ttlm_set_graph_replay(ttlm_model *model, int enabled);

/* State of the last step, for layer-by-layer checks (host outputs, each may be NULL):
 * x_in f32 [2880] = input of `layer` (the embedding for layer 0), residual f32 [2880]
 * after attention, indices int32 [4] / weights f32 [4] its routing. */
int ttlm_layer_state(ttlm_model *model, uint32_t layer, float *x_in, float *residual, int32_t *indices,
                     float *weights);
/* The final residual stream (input of the output norm) of the last step. */
int ttlm_final_state(ttlm_model *model, float *x_final);
/* Key and value caches of `layer`, positions [0, positions): f32 [positions][8][64] each. */
int ttlm_kv_cache(ttlm_model *model, uint32_t layer, uint32_t positions, float *keys, float *values);
/* Fills positions [0, positions) of every layer's key and value caches with N(0, 1)
 * values from the synthetic generator (stream = seed-derived, per layer), as if that
 * many tokens had been decoded: a decode step at `positions` then attends over a full
 * context without decoding it first (hardware counter runs, whose profilers serialize
 * every launch).  No reference counterpart. */
int ttlm_fill_kv_synthetic(ttlm_model *model, uint32_t positions, uint64_t seed);
/* Bytes of device memory the model holds. */
size_t ttlm_device_bytes(const ttlm_model *model);
/* Algorithmic bytes one decode step reads and writes at this position (weights actually
 * touched: 4 experts per layer, the attention span per layer, embedding row, unembedding). */
double ttlm_step_bytes(const ttlm_model *model, uint32_t position);

/* ---- text <-> tokens (ttlab::Tokenizer, tt-lab_amd/host/tokenizer.{hpp,cpp}) ----------
 * The gpt-oss byte-level BPE of a GGUF file's tokenizer.ggml.* metadata, as the
 * reference's Tokenizer (tokenizer.h:15-34, tokenizer.cpp:273-406); its constructor
 * sets LC_CTYPE from the environment, as the reference's does, and the letter, digit and
 * space classes of the pre-tokenizer follow that locale. */
typedef struct ttlm_tokenizer ttlm_tokenizer;
/* Tokenizer(file) (tokenizer.cpp:273-306): maps the file, checks the metadata. */
int ttlm_tokenizer_open(const char *gguf_path, ttlm_tokenizer **out);
void ttlm_tokenizer_free(ttlm_tokenizer *tokenizer);
/* Tokenizer::encode (tokenizer.cpp:308-331) of text[0, length): *count = the number of ids;
 * min(*count, capacity) of them are written to tokens. */
int ttlm_tokenizer_encode(const ttlm_tokenizer *tokenizer, const char *text, size_t length, int32_t *tokens,
                          size_t capacity, size_t *count);
/* Tokenizer::decode_to (tokenizer.cpp:370-401): the bytes of `token` into out[0, capacity),
 * *written of them; errors (an id out of range, a buffer too small) as the reference's. */
int ttlm_tokenizer_decode(const ttlm_tokenizer *tokenizer, int32_t token, int render_special, char *out,
                          size_t capacity, size_t *written);
/* Vocabulary size (tokenizer.ggml.tokens). */
size_t ttlm_tokenizer_vocabulary(const ttlm_tokenizer *tokenizer);
/* The gpt-4o pre-tokenizer's pieces of text[0, length) under the current LC_CTYPE
 * (tokenizer.cpp:112-237): *count pieces; ends[i] (i < capacity) is the byte offset where
 * piece i ends.  No reference counterpart as an entry point (the reference's is internal). */
int ttlm_pretokenize(const char *text, size_t length, size_t *ends, size_t capacity, size_t *count);
/* harmony_prompt (tokenizer.cpp:404-406) of user[0, length) into out[0, capacity); returns
 * the formatted length (the text is cut to capacity). */
size_t ttlm_harmony_prompt(const char *user, size_t length, char *out, size_t capacity);

#ifdef __cplusplus
}
#endif

#endif
