// ttlab::HipGptOssModel: the reference's GptOssModel decode loop (model.cpp:557-612)
// driving the gfx950 kernels through the C ABI.  One decode step is recorded once
// as a HIP graph; token and position live in device memory, so a step replays
// with no host work and feeds its own greedy token to the next step.
#include "gpt_oss_hip.hpp"

#include "gguf.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace ttlab {

namespace {

constexpr size_t kHidden = HipGptOssModel::embedding_length;
constexpr size_t kUsed = HipGptOssModel::experts_used;
constexpr size_t kQueryWidth = HipGptOssModel::query_heads * HipGptOssModel::head_size;  // 4096
constexpr size_t kKvWidth = HipGptOssModel::kv_heads * HipGptOssModel::head_size;        // 512
constexpr size_t kQkvRows = kQueryWidth + 2 * kKvWidth;                                  // 5120
constexpr size_t kSlidingWindow = 128;                                                    // model.h:44
constexpr size_t kPrefillBatch = 512;  // tokens per layer-major prefill pass
constexpr size_t kQ8RowBytes2880 = 2880 / 32 * 34;
constexpr size_t kQ8RowBytes4096 = 4096 / 32 * 34;
constexpr size_t kMxfp4RowBytes = 2880 / 32 * 17;

}  // namespace

void check(int status, const char *what) {
    if (status != TTL_OK) {
        throw std::runtime_error(std::string(what) + ": " + ttl_last_error());
    }
}

uint64_t synth_stream(int layer, uint32_t kind) {
    return uint64_t(int64_t(layer) + 1) * 100000u + uint64_t(kind) * 1000u;
}

std::array<float, 32> rope_frequencies() {
    // model.cpp:124-139 with the constants of model.h:38,46-50, in float as there.
    const float head_size = 64.0f, rope_base = 150000.0f, rope_scale = 1.0f / 32.0f;
    const float original_context = 4096.0f, beta_fast = 32.0f, beta_slow = 1.0f;
    const float pi = 3.14159265358979323846f;
    const float corr = head_size * std::log(original_context / (beta_fast * 2.0f * pi)) / (2.0f * std::log(rope_base));
    const float corr_slow =
        head_size * std::log(original_context / (beta_slow * 2.0f * pi)) / (2.0f * std::log(rope_base));
    const float low = std::max(0.0f, std::floor(corr));
    const float high = std::min(head_size - 1.0f, std::ceil(corr_slow));
    std::array<float, 32> f{};
    for (size_t pair = 0; pair < 32; ++pair) {
        const float dimension = float(pair * 2);
        const float theta_extrap = std::pow(rope_base, -dimension / head_size);
        const float y = (float(pair) - low) / std::max(0.001f, high - low);
        const float ramp = 1.0f - std::clamp(y, 0.0f, 1.0f);
        f[pair] = rope_scale * theta_extrap * (1.0f - ramp) + theta_extrap * ramp;
    }
    return f;
}

HipGptOssModel::HipGptOssModel(const SyntheticSpec &spec, int device) : spec_(spec) {
    if (spec.layers < 1 || spec.layers > 36) {
        throw std::runtime_error("layers must be 1..36");
    }
    if (spec.experts != 32 && spec.experts != 128) {
        throw std::runtime_error("unsupported expert count");  // model.cpp:94-97
    }
    if (spec.capacity < 1 || spec.capacity > context_length || spec.vocab < 1) {
        throw std::runtime_error("token capacity exceeds model context");  // model.cpp:99-101
    }
    check(ttl_create(device, &ctx_), "ttl_create");
    try {
        generate_weights();
        finish_construction();
    } catch (...) {
        release();
        throw;
    }
}

HipGptOssModel::HipGptOssModel(const GgufFile &file, size_t token_capacity, int device, bool strict)
    : HipGptOssModel(GgufSourceOf<GgufFile>(file), token_capacity, std::string(), 0, device, strict) {}

HipGptOssModel::HipGptOssModel(const GgufSource &file, size_t token_capacity, const std::string &dump_directory,
                               size_t batch_capacity, int device, bool strict) {
    const GgufModelShape shape = check_gguf_source(file, strict);
    // model.cpp:99-107, in the reference's order
    if (token_capacity > context_length) {
        throw std::runtime_error("token capacity exceeds model context");
    }
    if (batch_capacity > token_capacity) {
        throw std::runtime_error("batch capacity exceeds token capacity");
    }
    if (!dump_directory.empty()) {
        throw std::runtime_error("tensor dumps are not supported by the gfx950 backend");
    }
    if (token_capacity < 1) {
        // the reference builds a model without KV caches, which no forward can use
        throw std::runtime_error("the gfx950 backend needs a token capacity of at least 1");
    }
    spec_.layers = shape.layers;
    spec_.experts = shape.experts;
    spec_.vocab = shape.vocab;
    spec_.capacity = uint32_t(token_capacity);
    spec_.seed = 0;
    check(ttl_create(device, &ctx_), "ttl_create");
    try {
        upload_gguf(file);
        finish_construction();
    } catch (...) {
        release();
        throw;
    }
}

// RoPE table, activations and the captured step: the part of construction that does
// not depend on where the weights came from.
void HipGptOssModel::finish_construction() {
    for (const Layer &layer : layers_) {
        for (const ttl_mxfp4 *t : {layer.gate, layer.up, layer.down}) {
            if (ttl_mxfp4_edge_scales(t) != 0) {
                prefill_by_decode_ = true;  // the MFMA prefill refuses E8M0 0 / 255
            }
        }
    }
    {
        // RoPE coefficients per position and pair, as apply_rope computes them (model.cpp:230-245).
        const std::array<float, 32> f = rope_frequencies();
        const float magnitude = 1.0f + 0.1f * std::log(1.0f / (1.0f / 32.0f));
        std::vector<float> table(size_t(spec_.capacity) * 64);
        for (size_t pos = 0; pos < spec_.capacity; ++pos) {
            for (size_t pair = 0; pair < 32; ++pair) {
                const float theta = float(pos) * f[pair];
                table[pos * 64 + pair * 2] = std::cos(theta) * magnitude;
                table[pos * 64 + pair * 2 + 1] = std::sin(theta) * magnitude;
            }
        }
        rope_ = static_cast<float *>(alloc(sizeof(float) * table.size()));
        check(ttl_memcpy_h2d(ctx_, rope_, table.data(), sizeof(float) * table.size()), "ttl_memcpy_h2d");
    }
    {
        // activations (all sizes fixed at construction; nothing is allocated per token)
        const size_t L = spec_.layers;
        token_ = static_cast<int32_t *>(alloc(sizeof(int32_t)));
        position_ = static_cast<int32_t *>(alloc(sizeof(int32_t)));
        history_ = static_cast<int32_t *>(alloc(sizeof(int32_t) * spec_.capacity));
        x_ = static_cast<float *>(alloc(sizeof(float) * (L + 1) * kHidden));
        residual_ = static_cast<float *>(alloc(sizeof(float) * L * kHidden));
        down_ = static_cast<float *>(alloc(sizeof(float) * L * kUsed * kHidden));
        indices_ = static_cast<int32_t *>(alloc(sizeof(int32_t) * L * kUsed));
        weights_ = static_cast<float *>(alloc(sizeof(float) * L * kUsed));
        hidden_ = static_cast<float *>(alloc(sizeof(float) * kUsed * kHidden));
        query_ = static_cast<float *>(alloc(sizeof(float) * kQueryWidth));
        attended_ = static_cast<float *>(alloc(sizeof(float) * kQueryWidth));
        attn_workspace_ = static_cast<float *>(alloc(ttl_attention_workspace_bytes(spec_.capacity)));
        logits_ = static_cast<float *>(alloc(sizeof(float) * spec_.vocab));
        logits_workspace_ = alloc(ttl_logits_workspace_bytes(spec_.vocab));
        host_logits_.resize(spec_.vocab);

        // layer-major prefill buffers for chunks of up to kPrefillBatch tokens
        const size_t B = std::min<size_t>(kPrefillBatch, spec_.capacity);
        prefill_batch_ = B;
        prefill_tokens_ = static_cast<int32_t *>(alloc(sizeof(int32_t) * B));
        x_seq_ = static_cast<float *>(alloc(sizeof(float) * (L + 1) * B * kHidden));
        norm_seq_ = static_cast<float *>(alloc(sizeof(float) * B * kHidden));
        qkv_seq_ = static_cast<float *>(alloc(sizeof(float) * B * kQkvRows));
        q_seq_ = static_cast<float *>(alloc(sizeof(float) * B * kQueryWidth));
        attended_seq_ = static_cast<float *>(alloc(sizeof(float) * B * kQueryWidth));
        residual_seq_ = static_cast<float *>(alloc(sizeof(float) * B * kHidden));
        shift_seq_ = static_cast<int32_t *>(alloc(sizeof(int32_t) * B));
        gemm_workspace_bytes_ = std::max(ttl_matmul_q8_0_workspace_bytes(uint32_t(B), 2880),
                                         ttl_matmul_q8_0_workspace_bytes(uint32_t(B), 4096));
        gemm_workspace_ = alloc(gemm_workspace_bytes_);
        moe_workspace_bytes_ =
            ttl_moe_prefill_batch_workspace_bytes(uint32_t(B), uint32_t(spec_.experts), uint32_t(kUsed));
        moe_workspace_ = alloc(moe_workspace_bytes_);
        check(ttl_sync(ctx_), "ttl_sync");
        record_step();
    }
}

HipGptOssModel::~HipGptOssModel() {
    release();
}

void HipGptOssModel::release() {
    if (!ctx_) {
        return;
    }
    ttl_sync(ctx_);
    if (step_) {
        ttl_graph_free(step_);
        step_ = nullptr;
    }
    ttl_q8_free(ctx_, unembedding_q8_);
    unembedding_q8_ = nullptr;
    for (Layer &layer : layers_) {
        ttl_q8_free(ctx_, layer.qkv);
        ttl_q8_free(ctx_, layer.attn_output);
        ttl_mxfp4_free(ctx_, layer.gate);
        ttl_mxfp4_free(ctx_, layer.up);
        ttl_mxfp4_free(ctx_, layer.down);
    }
    layers_.clear();
    for (void *p : allocations_) {
        ttl_free(ctx_, p);
    }
    allocations_.clear();
    ttl_destroy(ctx_);
    ctx_ = nullptr;
}

void *HipGptOssModel::alloc(size_t bytes) {
    void *p = nullptr;
    check(ttl_malloc(ctx_, bytes, &p), "ttl_malloc");
    allocations_.push_back(p);
    device_bytes_ += bytes;
    return p;
}

void HipGptOssModel::generate_weights() {
    const uint64_t seed = spec_.seed;
    const size_t E = spec_.experts;
    auto normal = [&](int layer, uint32_t kind, size_t n, float mean, float sigma) {
        float *p = static_cast<float *>(alloc(sizeof(float) * n));
        check(ttl_synth_normal(ctx_, seed, synth_stream(layer, kind), 0, n, mean, sigma, p), "ttl_synth_normal");
        return p;
    };
    auto q8 = [&](const std::vector<std::pair<uint32_t, size_t>> &parts, int layer, size_t cols,
                  const int32_t *row_source) {
        size_t rows = 0;
        for (const auto &part : parts) {
            rows += part.second;
        }
        const size_t row_bytes = cols / 32 * 34;
        void *staging = nullptr;
        check(ttl_malloc(ctx_, rows * row_bytes, &staging), "ttl_malloc");
        size_t offset = 0;
        for (const auto &part : parts) {
            check(ttl_synth_q8_0_gguf(ctx_, seed, synth_stream(layer, part.first), 0, part.second * (cols / 32),
                                      static_cast<uint8_t *>(staging) + offset * row_bytes),
                  "ttl_synth_q8_0_gguf");
            offset += part.second;
        }
        ttl_q8 *t = nullptr;
        const int status = ttl_q8_upload_dev(ctx_, staging, uint32_t(rows), uint32_t(cols), row_source, &t);
        ttl_free(ctx_, staging);
        check(status, "ttl_q8_upload_dev");
        device_bytes_ += ttl_q8_bytes(t);
        return t;
    };
    auto mxfp4 = [&](int layer, uint32_t kind) {
        ttl_mxfp4 *t = nullptr;
        check(ttl_mxfp4_synthetic(ctx_, 2880, 2880, uint32_t(E), seed, synth_stream(layer, kind), 119, 125, &t),
              "ttl_mxfp4_synthetic");
        device_bytes_ += ttl_mxfp4_bytes(t);
        return t;
    };

    std::vector<int32_t> qkv_rows(kQkvRows);
    check(ttl_qkv_row_source(qkv_rows.data()), "ttl_qkv_row_source");
    layers_.resize(spec_.layers);
    for (size_t i = 0; i < spec_.layers; ++i) {
        const int l = int(i);
        Layer &layer = layers_[i];
        layer.attn_norm = normal(l, kAttnNorm, kHidden, 1.0f, 0.05f);
        layer.post_norm = normal(l, kPostNorm, kHidden, 1.0f, 0.05f);
        layer.qkv = q8({{kQuery, kQueryWidth}, {kKey, kKvWidth}, {kValue, kKvWidth}}, l, 2880, qkv_rows.data());
        layer.qkv_bias = normal(l, kQkvBias, kQkvRows, 0.0f, 0.05f);
        layer.attn_output = q8({{kAttnOutput, kHidden}}, l, 4096, nullptr);
        layer.attn_output_bias = normal(l, kAttnOutputBias, kHidden, 0.0f, 0.05f);
        layer.sinks = normal(l, kSinks, query_heads, 0.0f, 1.0f);
        layer.router = static_cast<float *>(alloc(sizeof(float) * E * kHidden));
        check(ttl_synth_normal_bf16(ctx_, seed, synth_stream(l, kRouter), 0, E * kHidden, 0.02f, layer.router),
              "ttl_synth_normal_bf16");
        layer.router_bias = normal(l, kRouterBias, E, 0.0f, 0.02f);
        layer.gate = mxfp4(l, kGate);
        layer.up = mxfp4(l, kUp);
        layer.down = mxfp4(l, kDown);
        layer.gate_bias = normal(l, kGateBias, E * kHidden, 0.0f, 0.05f);
        layer.up_bias = normal(l, kUpBias, E * kHidden, 0.0f, 0.05f);
        layer.down_bias = normal(l, kDownBias, E * kHidden, 0.0f, 0.05f);
        layer.key_cache = static_cast<float *>(alloc(sizeof(float) * spec_.capacity * kKvWidth));
        layer.value_cache = static_cast<float *>(alloc(sizeof(float) * spec_.capacity * kKvWidth));
        check(ttl_fill_bytes(ctx_, layer.key_cache, 0, sizeof(float) * spec_.capacity * kKvWidth), "fill");
        check(ttl_fill_bytes(ctx_, layer.value_cache, 0, sizeof(float) * spec_.capacity * kKvWidth), "fill");
        ttl_moe_layer &m = layer.moe;
        m.hidden = uint32_t(kHidden);
        m.expert_hidden = uint32_t(kHidden);
        m.experts = uint32_t(E);
        m.used = uint32_t(kUsed);
        m.router_weight = layer.router;
        m.router_bias = layer.router_bias;
        m.gate = layer.gate;
        m.gate_bias = layer.gate_bias;
        m.up = layer.up;
        m.up_bias = layer.up_bias;
        m.down = layer.down;
        m.down_bias = layer.down_bias;
        m.input_norm = layer.post_norm;  // model.cpp:590: the MoE reads rms_norm(residual)
        m.input_norm_epsilon = norm_epsilon;
    }
    embedding_ = static_cast<uint8_t *>(alloc(size_t(spec_.vocab) * kQ8RowBytes2880));
    check(ttl_synth_q8_0_gguf(ctx_, seed, synth_stream(-1, kEmbedding), 0, size_t(spec_.vocab) * 90, embedding_),
          "ttl_synth_q8_0_gguf");
    output_norm_ = normal(-1, kOutputNorm, kHidden, 1.0f, 0.05f);
    unembedding_ = static_cast<uint16_t *>(alloc(sizeof(uint16_t) * size_t(spec_.vocab) * kHidden));
    check(ttl_synth_bf16(ctx_, seed, synth_stream(-1, kUnembedding), 0, size_t(spec_.vocab) * kHidden, unembedding_),
          "ttl_synth_bf16");
}

// One decode step (model.cpp:567-602) as launches on the context's stream:
//   embedding; per layer: Q/K/V (+ attention norm, RoPE, KV store), attention,
//   output projection + residual, router (+ post-attention norm), gate/up +
//   SwiGLU, down + combine + residual; output norm + logits; greedy argmax
//   (writes the next token, advances the position).
// The input of layer l's QKV projection (l == layers: of the unembedding) as the
// staging computes it: for l > 0 the previous layer's output is never materialized
// by a kernel of its own -- the MoE combine and the residual add (model.cpp:323-337,
// 592-594) run in the consumer's staging, x_l = residual_{l-1} + (0 + w_0 d_0 + ...
// + w_3 d_3) in the reference's rank order, and workgroup 0 stores x_l for the
// state readers (and for the O projection's residual add).
ttl_stage_input HipGptOssModel::layer_input(size_t l, const float *norm_weight) const {
    ttl_stage_input in{};
    in.norm_weight = norm_weight;
    in.epsilon = norm_epsilon;
    if (l == 0) {
        in.base = x_;
        return in;
    }
    in.base = residual_ + (l - 1) * kHidden;
    in.add = down_ + (l - 1) * kUsed * kHidden;
    in.add_weights = weights_ + (l - 1) * kUsed;
    in.add_count = kUsed;
    in.sum_out = x_ + l * kHidden;
    return in;
}

int HipGptOssModel::enqueue_step() {
    const size_t L = spec_.layers;
    int status = ttl_embedding_q8_0(ctx_, embedding_, spec_.vocab, token_, x_);
    for (size_t l = 0; l < L && status == TTL_OK; ++l) {
        Layer &layer = layers_[l];
        const ttl_stage_input in = layer_input(l, layer.attn_norm);
        status = ttl_attn_qkv(ctx_, layer.qkv, layer.qkv_bias, &in, rope_, position_, spec_.capacity, query_,
                              layer.key_cache, layer.value_cache);
        if (status == TTL_OK) {
            status = ttl_attention_decode(ctx_, query_, layer.key_cache, layer.value_cache, layer.sinks, position_,
                                          spec_.capacity, uint32_t(l), attn_workspace_, attended_);
        }
        if (status == TTL_OK) {
            ttl_stage_input o{};
            o.base = attended_;
            status = ttl_matvec_q8_0(ctx_, layer.attn_output, layer.attn_output_bias, &o, x_ + l * kHidden,
                                     residual_ + l * kHidden);
        }
        if (status == TTL_OK) {
            status = ttl_moe_route_gateup(ctx_, &layer.moe, residual_ + l * kHidden, hidden_, indices_ + l * kUsed,
                                          weights_ + l * kUsed);
        }
        if (status == TTL_OK) {
            // the four experts' down projections (+ bias), one workgroup per (slot, tile);
            // the combine and the residual add run in the next consumer's staging.  (One
            // launch for gate/up and down, ttl_moe_route_gateup_down, made the step
            // slightly slower: its in-launch handoff costs about what this kernel
            // boundary does.)
            status = ttl_moe_down(ctx_, &layer.moe, hidden_, indices_ + l * kUsed, down_ + l * kUsed * kHidden);
        }
    }
    if (status == TTL_OK) {
        const ttl_stage_input f = layer_input(L, output_norm_);
        status = unembedding_q8_ ? ttl_logits_q8_0(ctx_, unembedding_q8_, spec_.vocab, &f, logits_, logits_workspace_)
                                 : ttl_logits_bf16(ctx_, unembedding_, spec_.vocab, &f, logits_, logits_workspace_);
    }
    if (status == TTL_OK) {
        status = ttl_argmax(ctx_, spec_.vocab, logits_workspace_, token_, position_, history_, spec_.capacity);
    }
    return status;
}

void HipGptOssModel::record_step() {
    check(ttl_capture_begin(ctx_), "ttl_capture_begin");
    const int status = enqueue_step();
    std::string error = status == TTL_OK ? "" : ttl_last_error();
    const int end = ttl_capture_end(ctx_, &step_);
    if (status != TTL_OK) {
        throw std::runtime_error("recording the decode step: " + error);
    }
    check(end, "ttl_capture_end");
}

void HipGptOssModel::validate(int32_t token, size_t position) const {
    // model.cpp:558-566
    if (position >= context_length) {
        throw std::runtime_error("model context is full");
    }
    if (position >= spec_.capacity) {
        throw std::runtime_error("position exceeds startup token capacity");
    }
    if (token < 0 || uint32_t(token) >= spec_.vocab) {
        throw std::runtime_error("input token is out of range");
    }
}

void HipGptOssModel::set_position(int32_t token, size_t position) {
    const int32_t state[2] = {token, int32_t(position)};
    check(ttl_memcpy_h2d(ctx_, token_, &state[0], sizeof(int32_t)), "ttl_memcpy_h2d");
    check(ttl_memcpy_h2d(ctx_, position_, &state[1], sizeof(int32_t)), "ttl_memcpy_h2d");
}

void HipGptOssModel::run_step() {
    if (use_graph_) {
        check(ttl_graph_launch(ctx_, step_), "ttl_graph_launch");
    } else {
        check(enqueue_step(), "decode step");
    }
}

const float *HipGptOssModel::forward(int32_t token, size_t position) {
    validate(token, position);
    set_position(token, position);
    run_step();
    check(ttl_memcpy_d2h(ctx_, host_logits_.data(), logits_, sizeof(float) * spec_.vocab), "ttl_memcpy_d2h");
    return host_logits_.data();
}

// One layer-major pass of GptOssModel::prefill (model.cpp:474-553) over the `count`
// tokens already in prefill_tokens_, at positions first .. first + count - 1.  The
// per-token results do not depend on how a prompt is cut into passes: each pass's
// attention reads the earlier positions' keys and values from the caches.
int HipGptOssModel::enqueue_prefill_chunk(size_t first, size_t count) {
    const size_t L = spec_.layers, B = prefill_batch_;
    const uint32_t n = uint32_t(count);
    int status = ttl_embedding_q8_0_batch(ctx_, embedding_, spec_.vocab, prefill_tokens_, n, x_seq_);
    for (size_t l = 0; l < L && status == TTL_OK; ++l) {
        Layer &layer = layers_[l];
        const float *x_in = x_seq_ + l * B * kHidden;
        float *x_out = x_seq_ + (l + 1) * B * kHidden;
        // the normalized rows' f16-plane shifts come with the norm, for the GEMM after it
        status = ttl_rms_norm_rows_shifts(ctx_, x_in, n, layer.attn_norm, norm_epsilon, norm_seq_, shift_seq_);
        if (status == TTL_OK) {
            status = ttl_matmul_q8_0_shifted(ctx_, layer.qkv, nullptr, norm_seq_, shift_seq_, n, nullptr, qkv_seq_,
                                             gemm_workspace_, gemm_workspace_bytes_);
        }
        if (status == TTL_OK) {
            status = ttl_qkv_rope_store(ctx_, qkv_seq_, n, uint32_t(first), layer.qkv_bias, rope_,
                                        uint32_t(spec_.capacity), q_seq_, layer.key_cache, layer.value_cache);
        }
        if (status == TTL_OK) {
            status = ttl_attention_prefill(ctx_, q_seq_, layer.key_cache, layer.value_cache, layer.sinks,
                                           uint32_t(first), n, uint32_t(spec_.capacity), uint32_t(l), attended_seq_);
        }
        if (status == TTL_OK) {
            // model.cpp:519-529: output projection, then residual = x + projected
            status = ttl_matmul_q8_0(ctx_, layer.attn_output, layer.attn_output_bias, attended_seq_, n, x_in,
                                     residual_seq_, gemm_workspace_, gemm_workspace_bytes_);
        }
        if (status == TTL_OK) {
            status = ttl_rms_norm_rows_shifts(ctx_, residual_seq_, n, layer.post_norm, norm_epsilon, norm_seq_,
                                              shift_seq_);
        }
        if (status == TTL_OK) {
            ttl_moe_layer moe = layer.moe;
            moe.input_norm = nullptr;  // moe_batch receives the normalized sequence (model.cpp:531)
            // x_{l+1} = residual + moe (model.cpp:545-553), the add in the MoE's combine
            status = ttl_moe_prefill_fused(ctx_, &moe, norm_seq_, shift_seq_, residual_seq_, n, x_out, nullptr,
                                           nullptr, moe_workspace_, moe_workspace_bytes_);
        }
    }
    if (status == TTL_OK) {
        // model.cpp:555-559: the logits of the last token
        ttl_stage_input f{};
        f.base = x_seq_ + (L * B + count - 1) * kHidden;
        f.norm_weight = output_norm_;
        f.epsilon = norm_epsilon;
        status = unembedding_q8_ ? ttl_logits_q8_0(ctx_, unembedding_q8_, spec_.vocab, &f, logits_, logits_workspace_)
                                 : ttl_logits_bf16(ctx_, unembedding_, spec_.vocab, &f, logits_, logits_workspace_);
    }
    return status;
}

const float *HipGptOssModel::prefill(const int32_t *tokens, size_t count) {
    // model.cpp:464-472
    if (count == 0) {
        throw std::runtime_error("prefill needs at least one token");
    }
    if (count > context_length) {
        throw std::runtime_error("model context is full");
    }
    if (count > spec_.capacity) {
        throw std::runtime_error("prefill exceeds startup batch capacity");
    }
    for (size_t p = 0; p < count; ++p) {
        validate(tokens[p], p);
    }
    if (prefill_by_decode_) {
        // Expert weights with E8M0 scale 0 or 255 have no exact bf16 form for the batched
        // MFMA kernels; the decode kernels take every scale, so the prompt runs token by
        // token (GptOssModel::forward at each position, model.cpp:557-602).
        const float *logits = nullptr;
        for (size_t p = 0; p < count; ++p) {
            logits = forward(tokens[p], p);
        }
        return logits;
    }
    for (size_t first = 0; first < count; first += prefill_batch_) {
        const size_t n = std::min(prefill_batch_, count - first);
        check(ttl_memcpy_h2d(ctx_, prefill_tokens_, tokens + first, sizeof(int32_t) * n), "ttl_memcpy_h2d");
        check(enqueue_prefill_chunk(first, n), "prefill");
    }
    check(ttl_memcpy_d2h(ctx_, host_logits_.data(), logits_, sizeof(float) * spec_.vocab), "ttl_memcpy_d2h");
    return host_logits_.data();
}

void HipGptOssModel::prefill_state(size_t layer, size_t count, float *x_in) const {
    if (layer > spec_.layers || count > prefill_batch_) {
        throw std::runtime_error("prefill_state: layer or count out of range");
    }
    if (prefill_by_decode_) {
        throw std::runtime_error("prefill_state: this model's prefill runs as decode steps (E8M0 scale 0 or 255)");
    }
    check(ttl_memcpy_d2h(ctx_, x_in, x_seq_ + layer * prefill_batch_ * kHidden, sizeof(float) * count * kHidden),
          "ttl_memcpy_d2h");
}

int32_t HipGptOssModel::greedy(const float *logits) const {
    // model.cpp:604-612
    const float *best = logits;
    for (size_t i = 1; i < spec_.vocab; ++i) {
        if (logits[i] > *best) {
            best = logits + i;
        }
    }
    return int32_t(best - logits);
}

std::vector<int32_t> HipGptOssModel::generate(int32_t token, size_t position, size_t steps) {
    validate(token, position);
    if (position + steps > spec_.capacity) {
        throw std::runtime_error("position exceeds startup token capacity");
    }
    set_position(token, position);
    for (size_t s = 0; s < steps; ++s) {
        run_step();
    }
    std::vector<int32_t> out(steps);
    if (steps) {
        check(ttl_memcpy_d2h(ctx_, out.data(), history_ + position, sizeof(int32_t) * steps), "ttl_memcpy_d2h");
    }
    return out;
}

double HipGptOssModel::time_decode(int32_t token, size_t position, size_t warmup, size_t steps) {
    validate(token, position);
    if (position + warmup + steps > spec_.capacity || steps == 0) {
        throw std::runtime_error("position exceeds startup token capacity");
    }
    set_position(token, position);
    for (size_t s = 0; s < warmup; ++s) {
        run_step();
    }
    check(ttl_sync(ctx_), "ttl_sync");
    check(ttl_timer_start(ctx_), "ttl_timer_start");
    for (size_t s = 0; s < steps; ++s) {
        run_step();
    }
    float ms = 0.0f;
    check(ttl_timer_stop(ctx_, &ms), "ttl_timer_stop");
    return double(ms) / double(steps);
}

double HipGptOssModel::time_expert_kernel(size_t reps) {
    // The gate/up + SwiGLU launch of every layer, with the routing of the last step,
    // replayed back to back: microseconds per launch.
    const auto enqueue = [this]() {
        int status = TTL_OK;
        for (size_t l = 0; l < spec_.layers && status == TTL_OK; ++l) {
            status = ttl_moe_gateup_swiglu(ctx_, &layers_[l].moe, residual_ + l * kHidden, indices_ + l * kUsed,
                                           hidden_);
        }
        return status;
    };
    ttl_graph *graph = nullptr;
    if (use_graph_) {
        check(ttl_capture_begin(ctx_), "ttl_capture_begin");
        const int status = enqueue();
        const std::string error = status == TTL_OK ? "" : ttl_last_error();
        check(ttl_capture_end(ctx_, &graph), "ttl_capture_end");
        if (status != TTL_OK) {
            ttl_graph_free(graph);
            throw std::runtime_error("recording the expert kernels: " + error);
        }
    }
    const auto run = [&]() {
        check(graph ? ttl_graph_launch(ctx_, graph) : enqueue(), "expert kernels");
    };
    float ms = 0.0f;
    try {
        for (int w = 0; w < 3; ++w) {
            run();
        }
        check(ttl_sync(ctx_), "ttl_sync");
        check(ttl_timer_start(ctx_), "ttl_timer_start");
        for (size_t r = 0; r < reps; ++r) {
            run();
        }
        check(ttl_timer_stop(ctx_, &ms), "ttl_timer_stop");
    } catch (...) {
        ttl_graph_free(graph);
        throw;
    }
    ttl_graph_free(graph);
    return double(ms) * 1000.0 / double(reps * spec_.layers);
}

double HipGptOssModel::time_kernel(uint32_t kind, size_t position, size_t reps, size_t *launches) {
    if (kind >= kKernelKinds) {
        throw std::runtime_error("time_kernel: unknown kernel kind");
    }
    if (position >= spec_.capacity || reps == 0) {
        throw std::runtime_error("time_kernel: position beyond the token capacity, or no repetitions");
    }
    // Scratch outputs, so the step's state (layer inputs, residuals, routing, caches) is
    // untouched; inputs are the last step's.
    std::vector<void *> scratch;
    const auto take = [&](size_t bytes) {
        void *p = nullptr;
        check(ttl_malloc(ctx_, bytes, &p), "ttl_malloc");
        scratch.push_back(p);
        return p;
    };
    const auto release_scratch = [&]() {
        (void)ttl_sync(ctx_);
        for (void *p : scratch) {
            (void)ttl_free(ctx_, p);
        }
    };
    ttl_graph *graph = nullptr;
    float ms = 0.0f;
    size_t count = 0;
    try {
        int32_t *pos = static_cast<int32_t *>(take(sizeof(int32_t)));
        const int32_t p32 = int32_t(position);
        check(ttl_memcpy_h2d(ctx_, pos, &p32, sizeof(p32)), "ttl_memcpy_h2d");
        const size_t cache_bytes = sizeof(float) * spec_.capacity * kKvWidth;
        float *q = static_cast<float *>(take(sizeof(float) * kQueryWidth));
        float *kc = kind == kKernelQkv ? static_cast<float *>(take(cache_bytes)) : nullptr;
        float *vc = kind == kKernelQkv ? static_cast<float *>(take(cache_bytes)) : nullptr;
        float *vec = static_cast<float *>(take(sizeof(float) * kUsed * kHidden));
        float *vec2 = kind == kKernelGateUpDown ? static_cast<float *>(take(sizeof(float) * kUsed * kHidden)) : nullptr;
        int32_t *idx = static_cast<int32_t *>(take(sizeof(int32_t) * kUsed));
        float *w = static_cast<float *>(take(sizeof(float) * kUsed));
        float *logits = kind == kKernelLogits ? static_cast<float *>(take(sizeof(float) * spec_.vocab)) : nullptr;
        void *logits_ws = kind == kKernelLogits ? take(ttl_logits_workspace_bytes(spec_.vocab)) : nullptr;
        const size_t L = spec_.layers;
        const auto enqueue = [&]() {
            int status = TTL_OK;
            count = 0;
            if (kind == kKernelLogits) {
                ttl_stage_input f = layer_input(L, output_norm_);
                f.sum_out = nullptr;
                count = 1;
                return unembedding_q8_ ? ttl_logits_q8_0(ctx_, unembedding_q8_, spec_.vocab, &f, logits, logits_ws)
                                       : ttl_logits_bf16(ctx_, unembedding_, spec_.vocab, &f, logits, logits_ws);
            }
            for (size_t l = 0; l < L && status == TTL_OK; ++l) {
                Layer &layer = layers_[l];
                switch (kind) {
                case kKernelQkv: {
                    ttl_stage_input in = layer_input(l, layer.attn_norm);
                    in.sum_out = nullptr;
                    status = ttl_attn_qkv(ctx_, layer.qkv, layer.qkv_bias, &in, rope_, pos, spec_.capacity, q, kc, vc);
                    ++count;
                    break;
                }
                case kKernelAttentionWindow:
                case kKernelAttentionFull:
                    if ((l % 2 == 0) == (kind == kKernelAttentionWindow)) {
                        status = ttl_attention_decode(ctx_, query_, layer.key_cache, layer.value_cache, layer.sinks,
                                                      pos, spec_.capacity, uint32_t(l), attn_workspace_, q);
                        ++count;
                    }
                    break;
                case kKernelOutputProjection: {
                    ttl_stage_input o{};
                    o.base = attended_;
                    status = ttl_matvec_q8_0(ctx_, layer.attn_output, layer.attn_output_bias, &o, x_ + l * kHidden,
                                             vec);
                    ++count;
                    break;
                }
                case kKernelRouterRows:
                case kKernelGateUpRouted:
                    // the routed gate/up ranks the rows the last router launch left in the
                    // context's scratch (the last layer's): the same work as in the step
                    status = ttl_moe_route_gateup_stages(ctx_, &layer.moe, residual_ + l * kHidden, vec, idx, w,
                                                         kind == kKernelRouterRows ? TTL_ROUTE_ROWS : TTL_ROUTE_GATEUP);
                    ++count;
                    break;
                case kKernelGateUpGiven:
                    status = ttl_moe_gateup_swiglu(ctx_, &layer.moe, residual_ + l * kHidden, indices_ + l * kUsed,
                                                   vec);
                    ++count;
                    break;
                case kKernelDown:
                    status = ttl_moe_down(ctx_, &layer.moe, hidden_, indices_ + l * kUsed, vec);
                    ++count;
                    break;
                case kKernelGateUpDown:
                    status = ttl_moe_route_gateup_down(ctx_, &layer.moe, residual_ + l * kHidden, vec, idx, w, vec2,
                                                       TTL_ROUTE_GATEUP_DOWN);
                    ++count;
                    break;
                }
            }
            return status;
        };
        if (use_graph_) {
            check(ttl_capture_begin(ctx_), "ttl_capture_begin");
            const int status = enqueue();
            const std::string error = status == TTL_OK ? "" : ttl_last_error();
            check(ttl_capture_end(ctx_, &graph), "ttl_capture_end");
            if (status != TTL_OK) {
                throw std::runtime_error("recording the kernels to time: " + error);
            }
        }
        const auto run = [&]() {
            check(graph ? ttl_graph_launch(ctx_, graph) : enqueue(), "timed kernels");
        };
        for (int r = 0; r < 3; ++r) {
            run();
        }
        check(ttl_sync(ctx_), "ttl_sync");
        check(ttl_timer_start(ctx_), "ttl_timer_start");
        for (size_t r = 0; r < reps; ++r) {
            run();
        }
        check(ttl_timer_stop(ctx_, &ms), "ttl_timer_stop");
    } catch (...) {
        ttl_graph_free(graph);
        release_scratch();
        throw;
    }
    ttl_graph_free(graph);
    release_scratch();
    if (launches) {
        *launches = count;
    }
    return count ? double(ms) * 1000.0 / double(reps * count) : 0.0;
}

void HipGptOssModel::layer_state(size_t layer, float *x_in, float *residual, int32_t *indices, float *weights) const {
    if (layer >= spec_.layers) {
        throw std::runtime_error("layer out of range");
    }
    if (x_in) {
        check(ttl_memcpy_d2h(ctx_, x_in, x_ + layer * kHidden, sizeof(float) * kHidden), "ttl_memcpy_d2h");
    }
    if (residual) {
        check(ttl_memcpy_d2h(ctx_, residual, residual_ + layer * kHidden, sizeof(float) * kHidden), "ttl_memcpy_d2h");
    }
    if (indices) {
        check(ttl_memcpy_d2h(ctx_, indices, indices_ + layer * kUsed, sizeof(int32_t) * kUsed), "ttl_memcpy_d2h");
    }
    if (weights) {
        check(ttl_memcpy_d2h(ctx_, weights, weights_ + layer * kUsed, sizeof(float) * kUsed), "ttl_memcpy_d2h");
    }
}

void HipGptOssModel::final_state(float *x_final) const {
    check(ttl_memcpy_d2h(ctx_, x_final, x_ + spec_.layers * kHidden, sizeof(float) * kHidden), "ttl_memcpy_d2h");
}

void HipGptOssModel::kv_cache(size_t layer, size_t positions, float *keys, float *values) const {
    if (layer >= spec_.layers || positions > spec_.capacity) {
        throw std::runtime_error("layer or positions out of range");
    }
    const size_t bytes = sizeof(float) * positions * kKvWidth;
    check(ttl_memcpy_d2h(ctx_, keys, layers_[layer].key_cache, bytes), "ttl_memcpy_d2h");
    check(ttl_memcpy_d2h(ctx_, values, layers_[layer].value_cache, bytes), "ttl_memcpy_d2h");
}

void HipGptOssModel::fill_kv_synthetic(size_t positions, uint64_t seed) {
    if (positions > spec_.capacity) {
        throw std::runtime_error("positions exceed the token capacity");
    }
    const size_t n = positions * kKvWidth;
    for (size_t l = 0; l < layers_.size(); ++l) {
        check(ttl_synth_normal(ctx_, seed, 2 * l, 0, n, 0.0f, 1.0f, layers_[l].key_cache), "ttl_synth_normal");
        check(ttl_synth_normal(ctx_, seed, 2 * l + 1, 0, n, 0.0f, 1.0f, layers_[l].value_cache), "ttl_synth_normal");
    }
    check(ttl_sync(ctx_), "ttl_sync");
}

double HipGptOssModel::step_bytes(size_t position) const {
    // Bytes a decode step must move: weights it reads (only the 4 routed experts), the
    // KV span each layer attends over, the cache entries it writes, one embedding row,
    // the unembedding, and the token-sized vectors (negligible, counted as 0).
    const double attention = double(kQkvRows) * kQ8RowBytes2880 + double(kHidden) * kQ8RowBytes4096 +
                             4.0 * (kQkvRows + kHidden + 64 + 2 * kHidden);
    const double router = double(spec_.experts) * kHidden * 4 + double(spec_.experts) * 4;
    const double experts = double(kUsed) * (3.0 * kHidden * kMxfp4RowBytes + 3.0 * kHidden * 4);
    const double unembedding = unembedding_q8_ ? double(spec_.vocab) * kQ8RowBytes2880 : double(spec_.vocab) * kHidden * 2;
    double total = double(kQ8RowBytes2880) + unembedding + kHidden * 4;
    for (size_t l = 0; l < spec_.layers; ++l) {
        const size_t first = (l % 2 == 0 && position + 1 > kSlidingWindow) ? position + 1 - kSlidingWindow : 0;
        const double span = double(position + 1 - first);
        total += attention + router + experts + span * kKvWidth * 4 * 2 + kKvWidth * 4 * 2;
    }
    return total;
}

}  // namespace ttlab
