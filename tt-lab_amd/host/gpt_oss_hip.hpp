// ttlab::HipGptOssModel -- the gpt-oss decode loop of the reference's GptOssModel
// (model.h:15-31, model.cpp:557-612) on the gfx950 backend.  Host code only: every
// device operation goes through the C ABI in include/ttlab_hip.h.
#pragma once

#include "gguf_source.hpp"
#include "ttlab_hip.h"

#include <array>
#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

namespace ttlab {

// Turns a C ABI status into the reference's error convention (std::runtime_error,
// model.cpp:209-228).
void check(int status, const char *what);

// Synthetic weights.  Tensor `kind` of layer l comes from generator stream
// synth_stream(l, kind) (model-wide tensors use l = -1); MXFP4 expert e of a
// tensor uses stream synth_stream(l, kind) + e.  Distributions:
//   norms N(1, 0.05); q/k/v/o Q8_0 (fp16 scale in [2^-12, 2^-11), int8 uniform);
//   biases N(0, 0.05); sinks N(0, 1); router bf16 N(0, 0.02), bias N(0, 0.02);
//   experts MXFP4 (E8M0 uniform 119..125, codes uniform); expert biases N(0, 0.05);
//   embedding Q8_0; unembedding bf16 (exponents 120..123).
enum SynthKind : uint32_t {
    kAttnNorm = 1,
    kPostNorm = 2,
    kQuery = 3,
    kKey = 4,
    kValue = 5,
    kQkvBias = 6,
    kAttnOutput = 7,
    kAttnOutputBias = 8,
    kSinks = 9,
    kRouter = 10,
    kRouterBias = 11,
    kGate = 12,
    kUp = 13,
    kDown = 14,
    kGateBias = 15,
    kUpBias = 16,
    kDownBias = 17,
    kEmbedding = 1,
    kOutputNorm = 2,
    kUnembedding = 3,
};
uint64_t synth_stream(int layer, uint32_t kind);

struct SyntheticSpec {
    uint32_t layers = 24;       // 24 (20b) or 36 (120b); tests use fewer
    uint32_t experts = 32;      // 32 (20b) or 128 (120b)
    uint32_t vocab = 201088;
    uint32_t capacity = 2112;   // token capacity of the KV caches
    uint64_t seed = 0x77000003;
};

// YaRN RoPE frequencies exactly as model.cpp:124-139 computes them.
std::array<float, 32> rope_frequencies();

class GgufFile;

// What a gpt-oss GGUF file holds, after the reference's metadata and tensor checks
// (GptOssModel's constructor, model.cpp:64-206, with its error messages).  strict
// applies the reference's limits exactly (24 or 36 layers, 32 or 128 experts, the
// 201088-token vocabulary, a Q8_0 output.weight); without it, any 1..36 layers,
// 1..128 experts, a vocabulary that is a multiple of 16 and a BF16 output.weight are
// also accepted (small test models and the bf16-unembedding configurations).
struct GgufModelShape {
    uint32_t layers = 0, experts = 0, vocab = 0;
    uint32_t output_type = 0;  // GGML type id of output.weight: 8 (Q8_0) or 30 (BF16)
};
GgufModelShape check_gguf_source(const GgufSource &file, bool strict);
// The same checks on any file class with the reference's accessors (ttlab::GgufFile,
// the reference's GgufFile).
template <class File>
GgufModelShape check_gguf_model(const File &file, bool strict) {
    return check_gguf_source(GgufSourceOf<File>(file), strict);
}

class HipGptOssModel {
  public:
    static constexpr size_t context_length = 131072;      // model.h:17
    static constexpr size_t embedding_length = 2880;      // model.h:34
    static constexpr size_t query_heads = 64, kv_heads = 8, head_size = 64;
    static constexpr size_t experts_used = 4;
    static constexpr float norm_epsilon = 1.0e-5f;

    explicit HipGptOssModel(const SyntheticSpec &spec, int device = 0);
    // The weights of a gpt-oss GGUF file (check_gguf_model), uploaded and repacked on
    // the device; the file may be closed afterwards.  token_capacity as the reference's
    // constructor (model.cpp:64, 99-101).
    HipGptOssModel(const GgufFile &file, size_t token_capacity, int device = 0, bool strict = true);
    // The reference's constructor (model.h:19-20) for any file class with its accessors
    // (the reference's own GgufFile included), so `GptOssModel model(file, capacity,
    // dump_directory, batch)` compiles against this class, with the reference's
    // capacity checks (model.cpp:99-107).  batch_capacity sizes the reference's prefill
    // buffers; the device prefill picks its own chunk and otherwise ignores it.  Tensor
    // dumps (dump_directory) are not part of this backend: a non-empty one throws, as
    // does a capacity of 0 (a model no forward could use).  device and strict follow
    // the reference's parameters, with its defaults.
    template <class File, class = std::enable_if_t<!std::is_base_of_v<GgufSource, File>>>
    explicit HipGptOssModel(const File &file, size_t token_capacity = 0, std::string dump_directory = {},
                            size_t batch_capacity = 0, int device = 0, bool strict = true)
        : HipGptOssModel(GgufSourceOf<File>(file), token_capacity, dump_directory, batch_capacity, device, strict) {}
    ~HipGptOssModel();
    HipGptOssModel(const HipGptOssModel &) = delete;
    HipGptOssModel &operator=(const HipGptOssModel &) = delete;

    // The reference's interface (model.h:26-30).
    const float *prefill(const int32_t *tokens, size_t count);
    const float *forward(int32_t token, size_t position);
    int32_t greedy(const float *logits) const;

    // Greedy decode with the token fed back on the device: `steps` tokens.
    std::vector<int32_t> generate(int32_t token, size_t position, size_t steps);
    // Milliseconds per device-resident decode step (HIP events around graph replays).
    double time_decode(int32_t token, size_t position, size_t warmup, size_t steps);
    // Microseconds per launch of the MXFP4 gate/up + SwiGLU kernel (all layers, the
    // last step's routing, replayed `reps` times; HIP events on the model's stream).
    double time_expert_kernel(size_t reps);
    // The decode step's kernels, one kind at a time (TTLM_KERNEL_* in ttlab_model.h).
    enum KernelKind : uint32_t {
        kKernelQkv = 0,
        kKernelAttentionWindow = 1,  // the even (sliding-window) layers
        kKernelAttentionFull = 2,    // the odd layers: partials + combine
        kKernelOutputProjection = 3,
        kKernelRouterRows = 4,
        kKernelGateUpRouted = 5,     // top-k ranking at its head, as the step runs it
        kKernelGateUpGiven = 6,      // the same kernel with the indices given
        kKernelDown = 7,             // the four experts' down projections (+ bias)
        kKernelLogits = 8,
        kKernelGateUpDown = 9,       // gate/up (ranking) and down in one launch; not the step's
        kKernelKinds = 10,
    };
    // Microseconds per launch (for kKernelAttentionFull: per partials + combine pair) of
    // every launch of `kind` one step at `position` makes, with the last step's inputs
    // and scratch outputs (the model's state is unchanged), captured as one graph and
    // replayed `reps` times between HIP events.  *launches = launches per replay.
    double time_kernel(uint32_t kind, size_t position, size_t reps, size_t *launches);

    // Decode steps replay the captured step graph (default) or launch its kernels
    // one by one on the model's stream (same kernels, same order).
    void set_graph_replay(bool enabled) {
        use_graph_ = enabled;
    }

    // Last step's state, for layer-by-layer checks.
    void layer_state(size_t layer, float *x_in, float *residual, int32_t *indices, float *weights) const;
    // The last prefill chunk's inputs of `layer` (layer == layers: the final stream),
    // f32 [count][2880] for its first `count` tokens.
    void prefill_state(size_t layer, size_t count, float *x_in) const;
    // Tokens a prefill processes per layer-major pass (longer prompts run in chunks).
    size_t prefill_batch() const {
        return prefill_batch_;
    }
    void final_state(float *x_final) const;
    void kv_cache(size_t layer, size_t positions, float *keys, float *values) const;
    // Positions [0, positions) of every layer's caches filled with N(0, 1) values.
    void fill_kv_synthetic(size_t positions, uint64_t seed);
    size_t device_bytes() const {
        return device_bytes_;
    }
    double step_bytes(size_t position) const;
    const SyntheticSpec &spec() const {
        return spec_;
    }

  private:
    struct Layer {
        float *attn_norm = nullptr, *post_norm = nullptr;
        ttl_q8 *qkv = nullptr;
        float *qkv_bias = nullptr;
        ttl_q8 *attn_output = nullptr;
        float *attn_output_bias = nullptr;
        float *sinks = nullptr;
        float *router = nullptr, *router_bias = nullptr;
        ttl_mxfp4 *gate = nullptr, *up = nullptr, *down = nullptr;
        float *gate_bias = nullptr, *up_bias = nullptr, *down_bias = nullptr;
        float *key_cache = nullptr, *value_cache = nullptr;
        ttl_moe_layer moe{};
    };

    HipGptOssModel(const GgufSource &file, size_t token_capacity, const std::string &dump_directory,
                   size_t batch_capacity, int device, bool strict);
    void *alloc(size_t bytes);
    void release();
    void generate_weights();
    void upload_gguf(const GgufSource &file);
    void finish_construction();
    int enqueue_step();
    ttl_stage_input layer_input(size_t layer, const float *norm_weight) const;
    int enqueue_prefill_chunk(size_t first, size_t count);
    void record_step();
    void run_step();
    void set_position(int32_t token, size_t position);
    void validate(int32_t token, size_t position) const;

    SyntheticSpec spec_;
    ttl_ctx *ctx_ = nullptr;
    std::vector<void *> allocations_;
    std::vector<Layer> layers_;
    size_t device_bytes_ = 0;
    uint8_t *embedding_ = nullptr;   // Q8_0, GGUF rows
    float *output_norm_ = nullptr;
    uint16_t *unembedding_ = nullptr;     // bf16 [vocab][2880] (synthetic configurations)
    ttl_q8 *unembedding_q8_ = nullptr;    // Q8_0 output.weight (GGUF models)
    float *rope_ = nullptr;          // [capacity][32][2]
    // activations
    int32_t *token_ = nullptr, *position_ = nullptr, *history_ = nullptr;
    float *x_ = nullptr;             // [layers + 1][2880]: layer inputs, then the final stream
    float *residual_ = nullptr;      // [layers][2880]
    float *down_ = nullptr;          // [layers][4][2880]: each layer's expert down outputs
    int32_t *indices_ = nullptr;     // [layers][4]
    float *weights_ = nullptr;       // [layers][4]
    float *hidden_ = nullptr, *query_ = nullptr, *attended_ = nullptr, *attn_workspace_ = nullptr;
    float *logits_ = nullptr;
    void *logits_workspace_ = nullptr;
    ttl_graph *step_ = nullptr;
    bool use_graph_ = true;
    std::vector<float> host_logits_;
    // layer-major prefill (model.cpp:463-555), chunks of prefill_batch_ tokens
    size_t prefill_batch_ = 0;
    bool prefill_by_decode_ = false;  // some expert tensor has E8M0 scale 0 or 255
    int32_t *prefill_tokens_ = nullptr;
    float *x_seq_ = nullptr;         // [layers + 1][batch][2880]
    float *norm_seq_ = nullptr, *qkv_seq_ = nullptr, *q_seq_ = nullptr, *attended_seq_ = nullptr;
    float *residual_seq_ = nullptr;
    int32_t *shift_seq_ = nullptr;   // [batch] f16-plane shifts of the normalized rows
    void *gemm_workspace_ = nullptr, *moe_workspace_ = nullptr;
    size_t gemm_workspace_bytes_ = 0, moe_workspace_bytes_ = 0;
};

}  // namespace ttlab
