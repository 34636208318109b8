/*
 * ttlab_hip.h -- C ABI of the MI355X (gfx950) backend for tt-lab's quantized decode path.
 *
 * This is the drop-in boundary.  Everything behind it is hand-written HIP for
 * gfx950 in tt-lab_amd/csrc/; everything above it (the C++ facade in
 * tt-lab_amd/host/, the tests, bench.py) sees plain pointers and sizes only.
 *
 * Conventions
 *  - Every entry point returns 0 (TTL_OK) or a negative TTL_ERR_* code; the
 *    message of the last failure on the calling thread is ttl_last_error().
 *    The C++ facade turns a non-zero code into std::runtime_error, the
 *    reference's error convention (model.cpp:209-228, main.cpp:414-417).
 *  - Pointers named *_dev are device pointers (from ttl_malloc or a tensor
 *    handle); all others are host pointers.
 *  - Work is queued in order on the context's stream and is asynchronous with
 *    respect to the host, except ttl_memcpy_d2h and ttl_sync, which wait.
 *  - Shapes are validated on the host before any launch; expert indices that
 *    live in device memory are bounds-checked by the kernels (an index out of
 *    range produces NaN outputs, never an out-of-bounds read).
 *  - One context owns one device and one stream; calls on one context must not
 *    overlap from several host threads (the reference is single-threaded,
 *    AGENTS.md:3).
 */
#ifndef TTLAB_HIP_H
#define TTLAB_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TTL_OK 0
#define TTL_ERR_INVALID -1   /* bad argument (null pointer, unsupported type)     */
#define TTL_ERR_SHAPE -2     /* shape the kernels do not support                  */
#define TTL_ERR_HIP -3       /* HIP runtime error (message has the HIP string)    */
#define TTL_ERR_NO_DEVICE -4 /* no gfx950 device at that ordinal                  */
#define TTL_ERR_MEMORY -5    /* device allocation failed                          */

typedef struct ttl_ctx ttl_ctx;
typedef struct ttl_mxfp4 ttl_mxfp4;

/* ---- context ---------------------------------------------------------------- */

/* Opens `device` (must be gfx950) and creates the context's stream.  No reference
 * counterpart: the reference CPU path has no device (the TT path's counterpart is
 * open_tt_firmware_runtime, tt_backend.cpp:1492-1528). */
int ttl_create(int device, ttl_ctx **out);
void ttl_destroy(ttl_ctx *ctx);
const char *ttl_last_error(void);
int ttl_sync(ttl_ctx *ctx);
/* Device name and compute-unit count, for reports. */
int ttl_device_info(ttl_ctx *ctx, char *name, size_t name_bytes, int *compute_units, double *hbm_bytes);

/* ---- device memory ------------------------------------------------------------ */

int ttl_malloc(ttl_ctx *ctx, size_t bytes, void **dev);
int ttl_free(ttl_ctx *ctx, void *dev);
int ttl_memcpy_h2d(ttl_ctx *ctx, void *dst_dev, const void *src, size_t bytes);
int ttl_memcpy_d2h(ttl_ctx *ctx, void *dst, const void *src_dev, size_t bytes);
int ttl_memcpy_d2d(ttl_ctx *ctx, void *dst_dev, const void *src_dev, size_t bytes);
/* Fills with a byte value using a kernel (safe inside HIP graph capture). */
int ttl_fill_bytes(ttl_ctx *ctx, void *dst_dev, uint8_t value, size_t bytes);

/* Reads `bytes` (a multiple of 16, 16-byte aligned) once with plain 16-byte loads
 * and no arithmetic: the streaming-read reference the matvec kernels are measured
 * against at the same bytes per launch.  Measurement only, with no counterpart in
 * the reference.  sink_dev (4 bytes) is written only if the XOR of one thread's
 * words equals a fixed constant. */
int ttl_stream_read(ttl_ctx *ctx, const void *src_dev, size_t bytes, uint32_t *sink_dev);

/* ttl_stream_read with ordinary loads instead of non-temporal ones (the kernels mark
 * their streamed weights non-temporal; this is the comparison).  Measurement only. */
int ttl_stream_read_plain(ttl_ctx *ctx, const void *src_dev, size_t bytes, uint32_t *sink_dev);

/* The cost of a kernel boundary: a graph of `launches` dependent kernels (blocks
 * workgroups of `threads` threads each), each reading in every workgroup a word the
 * previous kernel wrote, replayed 20 times; *us_per_kernel is the time per launch,
 * *wrong 1 if the chain's count came out wrong.  Measurement only, with no counterpart
 * in the reference: the fixed cost every kernel of the decode step pays. */
int ttl_measure_boundary(ttl_ctx *ctx, uint32_t launches, uint32_t blocks, uint32_t threads, float *us_per_kernel,
                         uint32_t *wrong);

/* The cost of handing 2880 floats from 180 producer workgroups to 32 consumer
 * workgroups, each consumer needing all of them: mode 0 across a kernel boundary (a
 * producer launch, then a consumer launch), mode 1 inside one launch (release fence and
 * a flag per producer, bounded polling, acquire fence), mode 2 inside one launch without
 * fences (values and flags written through with agent-scope stores after the values
 * completed, polled and read with agent-scope loads).  `launches` handoffs are
 * captured into a graph and replayed; *us_per_handoff is the average, *wrong the
 * consumers that read a wrong sum or gave up polling (0 when the handoff worked).
 * Measurement only, with no counterpart in the reference: it is why the decode step
 * keeps one kernel per dependency level. */
int ttl_measure_handoff(ttl_ctx *ctx, int mode, uint32_t launches, float *us_per_handoff, uint32_t *wrong);

/* ---- timing (HIP events on the context's stream) -------------------------------- */

int ttl_timer_start(ttl_ctx *ctx);
/* Records the stop event, waits for it, returns milliseconds since ttl_timer_start. */
int ttl_timer_stop(ttl_ctx *ctx, float *ms);

/* ---- synthetic inputs (same bits as the specification in oracle/ttlab_oracle.h) --- */

int ttl_synth_normal(ttl_ctx *ctx, uint64_t seed, uint64_t stream, size_t offset, size_t n, float mean,
                     float sigma, float *out_dev);
int ttl_synth_normal_bf16(ttl_ctx *ctx, uint64_t seed, uint64_t stream, size_t offset, size_t n, float sigma,
                          float *out_dev);
/* BF16 bit patterns (random sign and mantissa, exponent 120..123). */
int ttl_synth_bf16(ttl_ctx *ctx, uint64_t seed, uint64_t stream, size_t offset, size_t n, uint16_t *out_dev);
/* GGUF-layout MXFP4 blocks (17 B each), E8M0 uniform in [emin, emax]. */
int ttl_synth_mxfp4_gguf(ttl_ctx *ctx, uint64_t seed, uint64_t stream, size_t block_offset, size_t n,
                         uint32_t emin, uint32_t emax, uint8_t *out_dev);

/* ---- MXFP4 tensors ---------------------------------------------------------------- *
 * A ttl_mxfp4 holds `experts` matrices of `rows` x `cols` MXFP4 values, the GGUF
 * tensor {cols, rows, experts} of type 39 (tensor.h:15-17, model.cpp:160-169):
 * GGUF stores row r of expert e as cols/32 blocks of 17 bytes (E8M0 scale, then
 * 16 bytes of packed E2M1 codes; tensor.cpp:136-161, 283-296).  On upload the
 * blocks are repacked into two planes -- 16-byte code chunks and scale bytes --
 * tiled by 16 rows so one 64-lane load is 1 KiB of contiguous codes; the decode is
 * byte-identical.  Supported shapes: cols = 2880 (the reference's only width,
 * tensor.cpp:76-79), rows a multiple of 16.                                         */

int ttl_mxfp4_upload(ttl_ctx *ctx, const void *gguf_blocks, uint32_t rows, uint32_t cols, uint32_t experts,
                     ttl_mxfp4 **out);
/* Same, from GGUF-layout blocks already in device memory.  Waits for the repack: it
 * reads back whether any block has E8M0 scale 0 or 255 (ttl_mxfp4_edge_scales). */
int ttl_mxfp4_upload_dev(ttl_ctx *ctx, const void *gguf_blocks_dev, uint32_t rows, uint32_t cols,
                         uint32_t experts, ttl_mxfp4 **out);
/* Generates the tensor on the device: expert e is stream `stream + e` of the MXFP4
 * generator, so any expert can be regenerated on the host independently. */
int ttl_mxfp4_synthetic(ttl_ctx *ctx, uint32_t rows, uint32_t cols, uint32_t experts, uint64_t seed,
                        uint64_t stream, uint32_t emin, uint32_t emax, ttl_mxfp4 **out);
/* Writes the GGUF-layout bytes of the whole tensor back to host memory. */
int ttl_mxfp4_download(ttl_ctx *ctx, const ttl_mxfp4 *tensor, void *gguf_blocks);
void ttl_mxfp4_free(ttl_ctx *ctx, ttl_mxfp4 *tensor);
int ttl_mxfp4_shape(const ttl_mxfp4 *tensor, uint32_t *rows, uint32_t *cols, uint32_t *experts);
size_t ttl_mxfp4_bytes(const ttl_mxfp4 *tensor);
/* 1 if some block of the tensor has E8M0 scale 255, or scale 0 with a code of nonzero
 * magnitude, else 0 (negative: error).  The reference decodes those scales as 2^127 and
 * 2^-128 per integer unit (tensor.cpp:36-44); the matvec entry points do too.  The
 * batched MFMA entry points convert weights to bf16 with the scale folded in, which
 * has no exact form for them: ttl_matmul_mxfp4_selected refuses such an expert and
 * ttl_moe_prefill* such a tensor with TTL_ERR_SHAPE; HipGptOssModel then runs prefill
 * as decode steps. */
int ttl_mxfp4_edge_scales(const ttl_mxfp4 *tensor);
/* 1 if every block with a code of nonzero magnitude has E8M0 scale 114..140, so that every
 * weight E2M1 x 2^(e-127) is a normal f16, else 0 (negative: error).  Then the unscaled
 * prefill path (ttl_moe_prefill*) runs that tensor's GEMM on f16 MFMA with its f32 operand
 * (the down GEMM's SwiGLU hidden; gate/up's f32 tokens when both gate and up qualify) as
 * two f16 planes; otherwise on bf16 MFMA with it as three bf16 planes.  No reference
 * counterpart (a property of this backend's kernels). */
int ttl_mxfp4_f16_exact(const ttl_mxfp4 *tensor);

/* Decodes expert `expert` to f32 [rows][cols] on the device (out_dev).
 * mode 0: the reference's table, weight = 2^(e-128) * int(code) (tensor.cpp:34-74).
 * mode 1: the decode the matvec kernels perform: the gfx950 fp4 conversion
 *         instruction, then the block scale 2^(e-127) applied by ldexp.
 * mode 2: the decode the batched (MFMA) kernels perform: the gfx950 conversion to
 *         bf16 with the E8M0 scale folded in, widened to f32. */
int ttl_mxfp4_dequantize(ttl_ctx *ctx, const ttl_mxfp4 *tensor, uint32_t expert, int mode, float *out_dev);

/* y = W[expert] x + bias[expert].  Replaces matvec_add_mxfp4_2880
 * (tensor.h:28-35, tensor.cpp:239-304): bias_dev is f32 [experts][rows] (NULL for
 * none), x_dev f32 [cols], y_dev f32 [rows]. */
int ttl_matvec_mxfp4(ttl_ctx *ctx, const ttl_mxfp4 *w, const float *bias_dev, const float *x_dev, float *y_dev,
                     uint32_t expert);

/* Expert-indexed batch of matvecs in one launch: for slot s < n,
 * y[s] = W[experts[s]] x[s] + bias[experts[s]], reading only the selected experts.
 * experts_dev is int32 [n] in device memory (so router output feeds it without a
 * host round trip); x_dev is f32 [n][x_stride] (x_stride 0 = one shared x);
 * y_dev is f32 [n][rows].  The reference's callers loop over experts instead
 * (model.cpp:324-337). */
int ttl_matvec_mxfp4_experts(ttl_ctx *ctx, const ttl_mxfp4 *w, const float *bias_dev, const float *x_dev,
                             uint32_t x_stride, const int32_t *experts_dev, uint32_t n, float *y_dev);

/* ---- MoE decode (one token) ----------------------------------------------------- */

/* Router logits, top-k experts and their softmax weights.  Replaces the router
 * matvec_add_f32 call and the selection sort + softmax of GptOssModel::moe
 * (model.cpp:293-321, tensor.cpp:186-200).  weight_dev is f32 [experts][hidden]
 * (the GGUF ffn_gate_inp tensor), bias_dev f32 [experts], x_dev f32 [hidden].
 * Outputs: logits_dev f32 [experts], indices_dev int32 [k] (rank order, exactly the
 * reference's), weights_dev f32 [k].  hidden must be 2880, experts <= 192, k <= 16.
 * flags: TTL_ROUTER_FORCE_EXACT makes the kernel take its exact sequential path
 * (the path it otherwise takes only when a near-tie could change the selection). */
#define TTL_ROUTER_FORCE_EXACT 1u
int ttl_router_topk(ttl_ctx *ctx, const float *weight_dev, const float *bias_dev, uint32_t experts, uint32_t hidden,
                    const float *x_dev, uint32_t k, uint32_t flags, float *logits_dev, int32_t *indices_dev,
                    float *weights_dev);
/* Number of router launches on this context that took the exact sequential path. */
int ttl_router_exact_count(ttl_ctx *ctx, uint64_t *count);

/* One gpt-oss MoE layer's tensors, all in device memory (names as model.cpp:157-169). */
typedef struct {
    uint32_t hidden;             /* embedding length, 2880                        */
    uint32_t expert_hidden;      /* expert feed-forward length, 2880              */
    uint32_t experts;            /* 32 (20b) or 128 (120b)                        */
    uint32_t used;               /* experts per token, 4                          */
    const float *router_weight;  /* ffn_gate_inp.weight, f32 [experts][hidden]    */
    const float *router_bias;    /* ffn_gate_inp.bias, f32 [experts]              */
    const ttl_mxfp4 *gate;       /* ffn_gate_exps.weight: experts x expert_hidden x hidden */
    const float *gate_bias;      /* ffn_gate_exps.bias, f32 [experts][expert_hidden] (may be NULL) */
    const ttl_mxfp4 *up;         /* ffn_up_exps.weight                            */
    const float *up_bias;        /* ffn_up_exps.bias (may be NULL)                */
    const ttl_mxfp4 *down;       /* ffn_down_exps.weight: experts x hidden x expert_hidden */
    const float *down_bias;      /* ffn_down_exps.bias, f32 [experts][hidden] (may be NULL) */
    /* If non-NULL, x is the residual stream and the layer input is
     * rms_norm(x, input_norm, input_norm_epsilon) (post_attention_norm, model.cpp:590),
     * computed inside the router and gate/up kernels. */
    const float *input_norm;
    float input_norm_epsilon;
} ttl_moe_layer;

/* out = MoE(x) for one token: router + top-k + softmax, then for the k selected
 * experts only: gate and up matvecs with the clamped SwiGLU fused in, the down
 * matvec, and out = sum_r w_r * down_r in rank order.  Replaces GptOssModel::moe
 * (model.cpp:292-338).  indices_dev / weights_dev (int32 [used], f32 [used]) may be
 * NULL; when given they receive the routing. */
int ttl_moe_decode(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *x_dev, float *out_dev,
                   int32_t *indices_dev, float *weights_dev);

/* The stages of ttl_moe_decode, for callers that fuse the combine elsewhere.
 * gate/up + SwiGLU: hidden_dev f32 [used][expert_hidden] = swiglu(gate_e x + bg, up_e x + bu)
 *   for e = indices[r] (model.cpp:326-332);
 * down: down_dev f32 [used][hidden] = down_e hidden_r + bd (model.cpp:333);
 * combine: out = sum_r weights[r] * down_r, unfused, r = 0..k-1 (model.cpp:323,334-336). */
int ttl_moe_gateup_swiglu(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *x_dev,
                          const int32_t *indices_dev, float *hidden_dev);
/* Router + top-k + gate/up + SwiGLU (two launches: the router rows, then gate/up with
 * the certified top-k ranking at its head); writes hidden f32 [used][expert_hidden],
 * indices int32 [used] and weights f32 [used] (model.cpp:293-332). */
int ttl_moe_route_gateup(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *x_dev, float *hidden_dev,
                         int32_t *indices_dev, float *weights_dev);
/* ttl_moe_route_gateup split into its two launches, for callers that time them one
 * by one: TTL_ROUTE_ROWS computes the exact router rows into the context's scratch
 * (and, for a layer with an input norm, keeps the normalized input there),
 * TTL_ROUTE_GATEUP ranks the rows last computed on this context and runs gate/up on
 * that normalized input (x_dev itself for a layer without a norm).
 * No reference counterpart. */
#define TTL_ROUTE_ROWS 1u
#define TTL_ROUTE_GATEUP 2u
#define TTL_ROUTE_ALL 3u
int ttl_moe_route_gateup_stages(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *x_dev, float *hidden_dev,
                                int32_t *indices_dev, float *weights_dev, uint32_t stages);
int ttl_moe_down(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *hidden_dev, const int32_t *indices_dev,
                 float *down_dev);
/* GptOssModel::moe up to the combine (model.cpp:293-333) in two launches: the router
 * rows (TTL_ROUTE_ROWS, as above), then gate/up + SwiGLU and the `used` experts' down
 * rows + bias in one launch (TTL_ROUTE_GATEUP_DOWN): hidden_dev f32 [used][2880],
 * indices_dev int32 [used], weights_dev f32 [used], down_dev f32 [used][hidden].  Each
 * down workgroup issues its weight loads before waiting for its expert's hidden from the
 * gate/up workgroups of the same launch, so the down weights stream while gate/up ends.
 * The single launch needs its whole grid (used x 180 workgroups of 512 threads)
 * resident at once; where the occupancy does not allow it, gate/up and down run as two
 * launches with the same results (ttl_moe_gateup_down_fused says which).  The down sums
 * are the same products as ttl_moe_down's in another order.  Level with the two-launch
 * form on MI355X (16.7 against 10.5 + 5.8 us at the gpt-oss-20b shape) and slightly
 * slower in the decode step (1.207 against 1.193 ms per token), so the model's step does
 * not use it; kept for callers that cannot launch twice and as the measurement of that
 * choice.  No reference counterpart as one call. */
#define TTL_ROUTE_GATEUP_DOWN 4u
int ttl_moe_route_gateup_down(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *x_dev, float *hidden_dev,
                              int32_t *indices_dev, float *weights_dev, float *down_dev, uint32_t stages);
/* *fused = 1 if ttl_moe_route_gateup_down runs gate/up and down as one launch for this
 * layer shape on this device, 0 if as two. */
int ttl_moe_gateup_down_fused(ttl_ctx *ctx, const ttl_moe_layer *layer, int *fused);
/* Waits of the one-launch gate/up + down that ended at their bound since the context was
 * created (their down rows are NaN); 0 unless a workgroup of the grid was not resident. */
int ttl_moe_handoff_give_ups(ttl_ctx *ctx, uint64_t *count);
int ttl_moe_combine(ttl_ctx *ctx, const float *down_dev, const float *weights_dev, uint32_t k, uint32_t n,
                    float *out_dev);
/* down + combine + residual add in one launch (for used == 4; other counts run the
 * down and combine kernels): out = residual + (0 + w_0 d_0 + ... + w_{k-1} d_{k-1})
 * with d_r = down_e hidden_r + bd, in the reference's order (model.cpp:323-337,
 * 592-594).  residual_dev may be NULL (out = the MoE output); down_dev, if not NULL,
 * receives d (f32 [used][hidden]). */
int ttl_moe_down_combine(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *hidden_dev,
                         const int32_t *indices_dev, const float *weights_dev, const float *residual_dev,
                         float *out_dev, float *down_dev);

/* ---- batched prefill on MFMA (benchmark config 2) ------------------------------------ *
 * bf16 or f16 MFMA with f32 accumulation.  The weights E2M1 x 2^(e-127) are exact
 * bf16 values for E8M0 e in 1..254 (exact f16 values for e in 114..140, see
 * ttl_mxfp4_f16_exact); bf16 activations are one exact plane.  An f32 operand (f32
 * tokens, the SwiGLU hidden) is two f16 planes of x 2^k (k a power-of-two scale per
 * token, or 8 for the hidden; 22 of the value's 24 bits) where the tensor's scales
 * allow f16, else three bf16 planes that sum to it exactly; the sums are scaled back
 * by 2^-k before the bias.  Results agree with the reference's f32 sums to rounding
 * (relative L2 <= 1e-5), not bit for bit.
 * workspace_dev is caller-owned device memory, 256-byte aligned, of at least the
 * size the matching *_workspace_bytes function returns (workspace_bytes says how
 * much the caller holds; a smaller workspace is an error); calls sharing a
 * workspace must not overlap. */

#define TTL_DTYPE_F32 0
#define TTL_DTYPE_BF16 1
/* f32 / bf16 input computed on the scaled path (ttl_moe_prefill_experts): the
 * activations, and the SwiGLU hidden between the two GEMMs, quantized to MXFP8 (E4M3
 * values with an E8M0 exponent per 32-element block, the smallest exponent at which
 * the block's largest magnitude is at most 448 but never below -127, the smallest
 * E8M0 scale; round to nearest even), then
 * v_mfma_scale_f32_16x16x128_f8f6f4 with the MXFP4 weights as they are stored.  The
 * products are those of the dequantized values (ttl_mxfp8_dequantize), but the
 * instruction's accumulation is not exact in f32: within each 32-element block it
 * drops product bits below 2^-13 of the block's largest product (against the
 * reference's f32 sum of the same dequantized products: |err| up to 5.3e-6 of
 * sum |w x| per output; relative L2 7.9e-6 on normal activations, 1.6e-5 to 1.9e-5
 * on the SwiGLU hidden, whose blocks span a wider range).
 * The SwiGLU hidden is requantized too (its exponential and division on the
 * hardware's approximate instructions, a few ulp, ahead of the 3-bit rounding), so
 * the MoE's output carries the format's own error (relative L2 about 7e-2 on random
 * activations): the bf16 path stays the exact one.  No reference counterpart (the
 * reference computes in f32). */
#define TTL_DTYPE_F32_AS_MXFP8 2
#define TTL_DTYPE_BF16_AS_MXFP8 3

/* out[tokens[s]][r] = bias[expert][r] + sum_k W[expert][r][k] x[tokens[s]][k] for
 * s < count; other rows of out are untouched.  Replaces transpose_selected +
 * matmul_add_mxfp4_selected_transposed (tensor.h:38-51, tensor.cpp:306-495): the
 * reference transposes the selected rows of x on the host; here x_dev is the
 * untransposed f32 [x_rows][x_stride] and tokens_dev int32 [count] in device memory
 * (a token >= x_rows is skipped).  out_dev is f32 [x_rows][rows].  w->rows must be
 * a multiple of 192 (the reference's only shape is 2880). */
size_t ttl_matmul_mxfp4_selected_workspace_bytes(uint32_t count);
int ttl_matmul_mxfp4_selected(ttl_ctx *ctx, const ttl_mxfp4 *w, const float *bias_dev, const float *x_dev,
                              uint32_t x_stride, uint32_t x_rows, const int32_t *tokens_dev, uint32_t count,
                              float *out_dev, uint32_t expert, void *workspace_dev, size_t workspace_bytes);

/* ttl_matmul_mxfp4_selected on the scaled path: the selected tokens' rows quantized to
 * MXFP8 (see TTL_DTYPE_F32_AS_MXFP8), then v_mfma_scale with the MXFP4 weights; the
 * products are exactly those of ttl_mxfp8_dequantize's values, their sum is the
 * instruction's.  No reference counterpart (a faster, inexact form of
 * matmul_add_mxfp4_selected_transposed, tensor.cpp:306-495). */
size_t ttl_matmul_mxfp4_selected_mxfp8_workspace_bytes(uint32_t count);
int ttl_matmul_mxfp4_selected_mxfp8(ttl_ctx *ctx, const ttl_mxfp4 *w, const float *bias_dev, const float *x_dev,
                                    uint32_t x_stride, uint32_t x_rows, const int32_t *tokens_dev, uint32_t count,
                                    float *out_dev, uint32_t expert, void *workspace_dev, size_t workspace_bytes);
/* The values the scaled path multiplies: each 2880-wide row of x (f32 or bf16) in
 * 32-element blocks quantized to MXFP8 and widened back to f32 (exact); a block with a
 * non-finite value becomes NaN.  out_dev f32 [rows][2880].  No reference counterpart. */
int ttl_mxfp8_dequantize(ttl_ctx *ctx, const void *x_dev, int x_dtype, uint32_t rows, float *out_dev);

/* The expert half of GptOssModel::moe_batch (model.cpp:378-460) for `count` tokens
 * with given routing: indices_dev int32 [count][used] and weights_dev f32
 * [count][used] (rank order, as the router writes them).  Pairs are bucketed by
 * expert in the reference's order (expert, then token, then rank); per expert the
 * gate and up GEMMs with the clamped SwiGLU, then the down GEMM; then
 * out[p] = sum over p's experts in ascending expert index of w * down (unfused,
 * from 0; model.cpp:450-459).  x_dev is [count][2880] of x_dtype (TTL_DTYPE_F32 or
 * TTL_DTYPE_BF16); out_dev f32 [count][2880].  A token with an expert index out of
 * range gets NaN outputs.  Unlike the reference, buckets of at most 4 tokens also
 * take the GEMM (the reference switches to per-token matvecs there,
 * model.cpp:22,404; the two differ only in f32 rounding). */
size_t ttl_moe_prefill_workspace_bytes(uint32_t count, uint32_t experts, uint32_t used, int x_dtype);
int ttl_moe_prefill_experts(ttl_ctx *ctx, const ttl_moe_layer *layer, const void *x_dev, int x_dtype,
                            uint32_t count, const int32_t *indices_dev, const float *weights_dev, float *out_dev,
                            void *workspace_dev, size_t workspace_bytes);
/* The whole of GptOssModel::moe_batch (model.cpp:340-461) for `count` tokens: the F32
 * router per token (matmul_add_f32, model.cpp:341) with the exact top-k and softmax
 * of the decode router (the certified selection, else the reference's sequential
 * sums and selection sort), then ttl_moe_prefill_experts on f32 input.  x_dev is the
 * normalized MoE input f32 [count][2880] as moe_batch receives it (model.cpp:549-551),
 * so layer->input_norm must be NULL; indices_dev / weights_dev (int32 / f32
 * [count][used]) may be NULL, else they receive the routing. */
size_t ttl_moe_prefill_batch_workspace_bytes(uint32_t count, uint32_t experts, uint32_t used);
/* ttl_moe_prefill with two of the layer loop's neighbouring steps folded in:
 * x_shift_dev (int32 [count], or NULL) holds the f16-plane shifts of the rows of x as
 * ttl_rms_norm_rows_shifts writes them, so no launch computes them again; residual_dev
 * (f32 [count][2880], 16-byte aligned, or NULL) makes out = residual + the MoE output,
 * the residual add of model.cpp:545-551 (ttl_add of the two, bit for bit).  No reference
 * counterpart as one entry point. */
int ttl_moe_prefill_fused(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *x_dev, const int32_t *x_shift_dev,
                          const float *residual_dev, uint32_t count, float *out_dev, int32_t *indices_dev,
                          float *weights_dev, void *workspace_dev, size_t workspace_bytes);
int ttl_moe_prefill(ttl_ctx *ctx, const ttl_moe_layer *layer, const float *x_dev, uint32_t count, float *out_dev,
                    int32_t *indices_dev, float *weights_dev, void *workspace_dev, size_t workspace_bytes);

/* ttl_moe_prefill_experts split into its launches, for callers that time or
 * reorder them: the stages in `stages` run in this order, each reading what the
 * earlier stages left in the workspace (so a stage may be re-run alone after one
 * full call with the same arguments).  No reference counterpart. */
#define TTL_PREFILL_PLAN 1u     /* bucket the pairs by expert, cut 64-slot tiles      */
#define TTL_PREFILL_GATHER 2u   /* the tiles' activations as MFMA operand fragments   */
#define TTL_PREFILL_GATEUP 4u   /* gate and up GEMMs + clamped SwiGLU                  */
#define TTL_PREFILL_DOWN 8u     /* down GEMM, per slot                                 */
#define TTL_PREFILL_COMBINE 16u /* weighted sum per token in expert order              */
#define TTL_PREFILL_ALL 31u
int ttl_moe_prefill_stages(ttl_ctx *ctx, const ttl_moe_layer *layer, const void *x_dev, int x_dtype,
                           uint32_t count, const int32_t *indices_dev, const float *weights_dev, float *out_dev,
                           void *workspace_dev, size_t workspace_bytes, uint32_t stages);

/* What a ttl_moe_prefill_experts (or _stages) call left in its workspace, per (token,
 * rank) pair p = token * used + rank, for checking the stages one by one; call it
 * after that call with the same layer, x_dtype, count and workspace.  hidden_dev f32
 * [count * used][expert_hidden] receives the pair's clamped SwiGLU hidden as the down
 * GEMM reads it (on the scaled path its MXFP8 values; hidden_scales_dev, if non-NULL,
 * u8 [count * used][90] receives their E8M0 bytes), down_dev f32 [count * used][hidden]
 * the pair's down row with its bias, before the routing weight.  A pair with an
 * invalid expert index gets NaN rows.  The reference's moe_batch holds the same values
 * in its per-expert hidden and down buffers (model.cpp:415-447); no reference
 * counterpart as an entry point. */
int ttl_moe_prefill_intermediates(ttl_ctx *ctx, const ttl_moe_layer *layer, int x_dtype, uint32_t count,
                                  const void *workspace_dev, size_t workspace_bytes, float *hidden_dev,
                                  float *down_dev, uint8_t *hidden_scales_dev);

/* ---- matvec inputs ----------------------------------------------------------------- *
 * The vector a matvec reads, with the elementwise steps GptOssModel::forward runs
 * before it fused in (each workgroup recomputes them; nothing is launched for them):
 *   v  = base + sum_r add_weights[r] * add[r]   (the MoE combine and residual add,
 *                                                model.cpp:323-337 and 592-594; add may be NULL)
 *   in = rms_norm(v, norm_weight, epsilon)      (tensor.cpp:568-580; norm_weight may be NULL)
 * sum_out, if non-NULL, receives v (the next residual stream value).  All pointers
 * are device pointers, 16-byte aligned. */
typedef struct {
    const float *base;
    const float *add;            /* f32 [add_count][n] or NULL */
    const float *add_weights;    /* f32 [add_count]            */
    uint32_t add_count;
    const float *norm_weight;    /* f32 [n] or NULL            */
    float epsilon;
    float *sum_out;              /* f32 [n] or NULL            */
} ttl_stage_input;

/* ---- Q8_0 tensors and the attention-side matvecs ----------------------------------- *
 * A ttl_q8 holds rows x cols Q8_0 values (GGUF type 8: per 32 values an fp16 scale
 * and 32 int8, tensor.cpp:94-114, 136-157), repacked on upload into 16-row tiles.
 * row_source (host, may be NULL) maps each repacked row to the GGUF row that fills
 * it, so several GGUF tensors can be stacked and reordered into one.  cols must be
 * 2880 or 4096, rows a multiple of 16. */
typedef struct ttl_q8 ttl_q8;
int ttl_q8_upload(ttl_ctx *ctx, const void *gguf_blocks, uint32_t rows, uint32_t cols, const int32_t *row_source,
                  uint32_t source_rows, ttl_q8 **out);
int ttl_q8_upload_dev(ttl_ctx *ctx, const void *gguf_blocks_dev, uint32_t rows, uint32_t cols,
                      const int32_t *row_source, ttl_q8 **out);
/* GGUF bytes of the repacked rows, in repacked row order. */
int ttl_q8_download(ttl_ctx *ctx, const ttl_q8 *tensor, void *gguf_blocks);
void ttl_q8_free(ttl_ctx *ctx, ttl_q8 *tensor);
size_t ttl_q8_bytes(const ttl_q8 *tensor);
/* GGUF Q8_0 blocks from the synthetic generator (oracle orc_synth_q8_0). */
int ttl_synth_q8_0_gguf(ttl_ctx *ctx, uint64_t seed, uint64_t stream, size_t block_offset, size_t n,
                        uint8_t *out_dev);

/* y = W in (+ bias) (+ residual).  Replaces matvec_q8_0 / matvec_add_q8_0
 * (tensor.h:26-27, tensor.cpp:202-237); with residual_dev it is the output
 * projection plus residual add of model.cpp:584-588. */
int ttl_matvec_q8_0(ttl_ctx *ctx, const ttl_q8 *w, const float *bias_dev, const ttl_stage_input *in,
                    const float *residual_dev, float *y_dev);

/* matmul_add_q8_0 (tensor.h:36-37, tensor.cpp:529-566) for `tokens` tokens, as
 * GptOssModel::prefill runs the attention projections (model.cpp:493-498, 519-520):
 * out[t][r] = bias[r] + sum_k W[r][k] x[t][k] (+ residual[t][r] when residual_dev is
 * non-NULL, the residual add of model.cpp:521-529).  x_dev f32 [tokens][cols] (cols
 * 2880 or 4096), out_dev f32 [tokens][rows] in the tensor's row order; bias_dev may
 * be NULL.  f16 MFMA (int8 codes, exact; each token's activations times a power of two
 * 2^k as two f16 planes, 22 of their 24 bits, the sums scaled back by 2^-k before the
 * bias) and the block scale applied per block: results agree with the reference to
 * f32 rounding.  workspace_dev (16-byte aligned) holds
 * ttl_matmul_q8_0_workspace_bytes(tokens, cols). */
size_t ttl_matmul_q8_0_workspace_bytes(uint32_t tokens, uint32_t cols);
int ttl_matmul_q8_0(ttl_ctx *ctx, const ttl_q8 *w, const float *bias_dev, const float *x_dev, uint32_t tokens,
                    const float *residual_dev, float *out_dev, void *workspace_dev, size_t workspace_bytes);
/* ttl_matmul_q8_0 with the tokens' f16-plane shifts given: shift_dev int32 [tokens] as
 * ttl_rms_norm_rows_shifts writes them for x, so no launch computes them again (the same
 * results, bit for bit).  No reference counterpart as an entry point. */
int ttl_matmul_q8_0_shifted(ttl_ctx *ctx, const ttl_q8 *w, const float *bias_dev, const float *x_dev,
                            const int32_t *shift_dev, uint32_t tokens, const float *residual_dev, float *out_dev,
                            void *workspace_dev, size_t workspace_bytes);

/* The row order ttl_attn_qkv expects of its 5120-row tensor: rows of attn_q (0..4095),
 * attn_k (4096..4607) and attn_v (4608..5119) stacked, reordered so each RoPE pair
 * (d, d+32) of a head shares a tile.  Fills row_source[5120]. */
int ttl_qkv_row_source(int32_t *row_source);

/* Q/K/V projection of one decode token (model.cpp:572-582): in is normally the
 * residual stream with the attention norm; bias_dev is f32 [5120] = q|k|v biases in
 * GGUF order; rope_dev is f32 [capacity][32][2] = (cos, sin) * (1 + 0.1 ln 32) per
 * position and pair, computed on the host exactly as apply_rope does (model.cpp:230-245);
 * position_dev is int32 [1].  Writes q (after RoPE) to q_dev f32 [4096] and k (after
 * RoPE), v to the caches f32 [capacity][8][64] at the position. */
int ttl_attn_qkv(ttl_ctx *ctx, const ttl_q8 *qkv, const float *bias_dev, const ttl_stage_input *in,
                 const float *rope_dev, const int32_t *position_dev, uint32_t capacity, float *q_dev,
                 float *k_cache_dev, float *v_cache_dev);

/* ---- attention with sinks --------------------------------------------------------- */

size_t ttl_attention_workspace_bytes(uint32_t capacity);
/* attention_from_cache (model.cpp:255-290) for the position in position_dev: even
 * layer_index uses the last 128 positions, odd all; sinks_dev f32 [64]; out_dev
 * f32 [4096].  workspace_dev holds ttl_attention_workspace_bytes(capacity). */
int ttl_attention_decode(ttl_ctx *ctx, const float *q_dev, const float *k_cache_dev, const float *v_cache_dev,
                         const float *sinks_dev, const int32_t *position_dev, uint32_t capacity, uint32_t layer_index,
                         float *workspace_dev, float *out_dev);

/* ttl_attention_decode without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  The full-context partials go to a
 * static device array of 4,325,376 bytes per GPU (held until the process ends), so
 * capacity is at most 16384 positions (larger is TTL_ERR_SHAPE).  Same kernels and
 * results as ttl_attention_decode.  Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (other streams or contexts) race. */
int ttl_attention_decode_noalloc(ttl_ctx *ctx, const float *q_dev, const float *k_cache_dev,
                                 const float *v_cache_dev, const float *sinks_dev, const int32_t *position_dev,
                                 uint32_t capacity, uint32_t layer_index, float *out_dev);

/* attention_from_cache (model.cpp:255-290) for `tokens` tokens at positions
 * first_position .. first_position + tokens - 1, as GptOssModel::prefill runs it per
 * token (model.cpp:510-514): q_dev / out_dev f32 [tokens][4096]; the caches must hold
 * every position up to the last token's.  Needs no workspace: each workgroup takes 16
 * tokens of one kv head and streams their positions through LDS with an online softmax. */
int ttl_attention_prefill(ttl_ctx *ctx, const float *q_dev, const float *k_cache_dev, const float *v_cache_dev,
                          const float *sinks_dev, uint32_t first_position, uint32_t tokens, uint32_t capacity,
                          uint32_t layer_index, float *out_dev);

/* ---- batched prefill helpers (GptOssModel::prefill, model.cpp:463-555) ------------- */

/* rms_norm (tensor.cpp:568-580) of each of `rows` rows of 2880 (model.cpp:487-491,
 * 524-526), in the decode kernels' summation order. */
int ttl_rms_norm_rows(ttl_ctx *ctx, const float *x_dev, uint32_t rows, const float *weight_dev, float epsilon,
                      float *out_dev);
/* ttl_rms_norm_rows that also writes each normalized row's f16-plane shift into
 * shift_dev (int32 [rows]; NULL: none): k = 15 - e for the row's largest finite
 * magnitude m = f 2^e, f in [0.5, 1) (0 for a row with no nonzero finite value), the
 * shift with which ttl_matmul_q8_0 and ttl_moe_prefill split a row into two f16
 * planes.  For ttl_matmul_q8_0_shifted and ttl_moe_prefill_fused; no reference
 * counterpart. */
int ttl_rms_norm_rows_shifts(ttl_ctx *ctx, const float *x_dev, uint32_t rows, const float *weight_dev,
                             float epsilon, float *out_dev, int32_t *shift_dev);
/* The bias, RoPE and KV-cache store of model.cpp:499-507 for `tokens` tokens at
 * positions first_position .. : qkv_dev f32 [tokens][5120] is the output of
 * ttl_matmul_q8_0 on a tensor in ttl_qkv_row_source order without its bias; bias_dev
 * f32 [5120] in GGUF order (attn_q, attn_k, attn_v biases); rope_dev as for
 * ttl_attn_qkv; q_dev f32 [tokens][4096]. */
int ttl_qkv_rope_store(ttl_ctx *ctx, const float *qkv_dev, uint32_t tokens, uint32_t first_position,
                       const float *bias_dev, const float *rope_dev, uint32_t capacity, float *q_dev,
                       float *k_cache_dev, float *v_cache_dev);
/* out = a + b elementwise over n floats (the residual adds of model.cpp:521-529,
 * 545-551). */
int ttl_add(ttl_ctx *ctx, const float *a_dev, const float *b_dev, size_t n, float *out_dev);

/* ---- embedding, unembedding, greedy ------------------------------------------------ */

/* load_token_embedding_q8_0 (tensor.cpp:171-184) for the token in token_dev; table_dev
 * holds the GGUF Q8_0 token_embd rows (vocab x 2880).  An out-of-range token gives NaNs. */
int ttl_embedding_q8_0(ttl_ctx *ctx, const void *table_dev, uint32_t vocab, const int32_t *token_dev,
                       float *out_dev);
/* The embeddings of `count` tokens (model.cpp:474-482): out_dev f32 [count][2880]. */
int ttl_embedding_q8_0_batch(ttl_ctx *ctx, const void *table_dev, uint32_t vocab, const int32_t *tokens_dev,
                             uint32_t count, float *out_dev);
size_t ttl_logits_workspace_bytes(uint32_t vocab);
/* logits = W in for a bf16 unembedding W [vocab][2880] (the synthetic configurations'
 * output.weight; the reference's is Q8_0, model.cpp:598-599), and per-group argmax
 * partials in workspace_dev for ttl_argmax. */
int ttl_logits_bf16(ttl_ctx *ctx, const uint16_t *weight_dev, uint32_t vocab, const ttl_stage_input *in,
                    float *logits_dev, void *workspace_dev);
/* The same for a Q8_0 unembedding (a GGUF model's output.weight, vocab x 2880;
 * matvec_q8_0 at model.cpp:598-599).  The partials feed ttl_argmax as those of
 * ttl_logits_bf16 do. */
int ttl_logits_q8_0(ttl_ctx *ctx, const ttl_q8 *weight, uint32_t vocab, const ttl_stage_input *in, float *logits_dev,
                    void *workspace_dev);
/* greedy (model.cpp:604-612) from ttl_logits_bf16's partials: writes the token to
 * token_dev and, if position_dev is non-NULL, also history_dev[position] (when
 * history_dev is non-NULL and position < history_len) and increments the position. */
int ttl_argmax(ttl_ctx *ctx, uint32_t vocab, const void *workspace_dev, int32_t *token_dev, int32_t *position_dev,
               int32_t *history_dev, uint32_t history_len);

/* ---- HIP graphs ------------------------------------------------------------------- *
 * Calls made on the context between ttl_capture_begin and ttl_capture_end are
 * recorded (not run) into a graph that ttl_graph_launch replays on the stream.
 * Only launch-only entry points may be captured (no ttl_memcpy_h2d/d2h, ttl_sync,
 * tensor uploads).  No reference counterpart (the reference runs on the CPU). */
typedef struct ttl_graph ttl_graph;
int ttl_capture_begin(ttl_ctx *ctx);
int ttl_capture_end(ttl_ctx *ctx, ttl_graph **out);
int ttl_graph_launch(ttl_ctx *ctx, ttl_graph *graph);
void ttl_graph_free(ttl_graph *graph);

#ifdef __cplusplus
}
#endif

#endif
