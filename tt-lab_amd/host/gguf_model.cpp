// Loading a gpt-oss GGUF file into ttlab::HipGptOssModel: the reference's checks
// (GptOssModel's constructor, model.cpp:64-206) and the uploads to the device.
#include "gguf.hpp"
#include "gpt_oss_hip.hpp"

#include <cmath>
#include <cstring>
#include <initializer_list>
#include <string>
#include <vector>

namespace ttlab {
namespace {

constexpr uint64_t kHidden = 2880, kQueryWidth = 4096, kKvWidth = 512, kQkvRows = kQueryWidth + 2 * kKvWidth;
constexpr uint64_t kLayerCapacity = 36, kExpertCapacity = 128, kVocabulary = 201088;

// require_integer / require_number (model.cpp:24-34)
void require_integer(const GgufSource &file, const char *key, uint64_t expected) {
    if (file.integer(key) != expected) {
        throw std::runtime_error("unsupported " + std::string(key));
    }
}
void require_number(const GgufSource &file, const char *key, double expected) {
    if (file.number(key) != expected) {
        throw std::runtime_error("unsupported " + std::string(key));
    }
}

// require_tensor (model.cpp:209-228)
TensorRef require_tensor(const GgufSource &file, const std::string &name, uint32_t type,
                         std::initializer_list<uint64_t> shape) {
    TensorRef t;
    if (!file.tensor(name, &t)) {
        throw std::runtime_error("missing tensor " + name);
    }
    if (t.type != type) {
        throw std::runtime_error("wrong type for tensor " + name);
    }
    if (t.dims != shape.size()) {
        throw std::runtime_error("wrong rank for tensor " + name);
    }
    size_t i = 0;
    for (uint64_t expected : shape) {
        if (t.shape[i++] != expected) {
            throw std::runtime_error("wrong shape for tensor " + name);
        }
    }
    return t;
}

// A tensor check_gguf_source() has already required.
TensorRef checked_tensor(const GgufSource &file, const std::string &name) {
    TensorRef t;
    if (!file.tensor(name, &t)) {
        throw std::runtime_error("missing tensor " + name);
    }
    return t;
}

std::string layer_prefix(size_t l) {
    return "blk." + std::to_string(l) + ".";
}

}  // namespace

GgufModelShape check_gguf_source(const GgufSource &file, bool strict) {
    if (file.string("general.architecture") != "gpt-oss") {
        throw std::runtime_error("model architecture is not gpt-oss");
    }
    const uint64_t layers = file.integer("gpt-oss.block_count");
    if (strict ? (layers != 24 && layers != 36) : (layers < 1 || layers > kLayerCapacity)) {
        throw std::runtime_error("only gpt-oss-20b and gpt-oss-120b are supported");
    }
    require_integer(file, "gpt-oss.context_length", HipGptOssModel::context_length);
    require_integer(file, "gpt-oss.embedding_length", kHidden);
    require_integer(file, "gpt-oss.feed_forward_length", kHidden);
    require_integer(file, "gpt-oss.attention.head_count", HipGptOssModel::query_heads);
    require_integer(file, "gpt-oss.attention.head_count_kv", HipGptOssModel::kv_heads);
    require_integer(file, "gpt-oss.attention.key_length", HipGptOssModel::head_size);
    require_integer(file, "gpt-oss.attention.value_length", HipGptOssModel::head_size);
    require_integer(file, "gpt-oss.expert_used_count", HipGptOssModel::experts_used);
    require_integer(file, "gpt-oss.expert_feed_forward_length", kHidden);
    require_integer(file, "gpt-oss.attention.sliding_window", 128);
    require_number(file, "gpt-oss.attention.layer_norm_rms_epsilon", double(HipGptOssModel::norm_epsilon));
    require_number(file, "gpt-oss.rope.freq_base", double(150000.0f));
    require_number(file, "gpt-oss.rope.scaling.factor", 32.0);
    require_integer(file, "gpt-oss.rope.scaling.original_context_length", 4096);
    require_number(file, "gpt-oss.rope.scaling.yarn_beta_fast", double(32.0f));
    require_number(file, "gpt-oss.rope.scaling.yarn_beta_slow", double(1.0f));
    const uint64_t experts = file.integer("gpt-oss.expert_count");
    if (strict ? (experts != 32 && experts != kExpertCapacity)
               : (experts < HipGptOssModel::experts_used || experts > kExpertCapacity)) {
        throw std::runtime_error("unsupported expert count");
    }

    GgufModelShape shape;
    shape.layers = uint32_t(layers);
    shape.experts = uint32_t(experts);
    TensorRef embd;
    uint64_t vocab = kVocabulary;
    if (!strict && file.tensor("token_embd.weight", &embd) && embd.dims == 2) {
        vocab = embd.shape[1];
        if (vocab < 16 || vocab % 16 != 0 || vocab > (1ull << 31)) {
            throw std::runtime_error("wrong shape for tensor token_embd.weight");
        }
    }
    shape.vocab = uint32_t(vocab);
    require_tensor(file, "token_embd.weight", kGgmlQ8_0, {kHidden, vocab});
    require_tensor(file, "output_norm.weight", kGgmlF32, {kHidden});
    TensorRef out;
    const uint32_t out_type = (!strict && file.tensor("output.weight", &out) && out.type == kGgmlBf16) ? kGgmlBf16
                                                                                                       : kGgmlQ8_0;
    require_tensor(file, "output.weight", out_type, {kHidden, vocab});
    shape.output_type = out_type;
    for (size_t l = 0; l < layers; ++l) {
        const std::string p = layer_prefix(l);
        require_tensor(file, p + "attn_norm.weight", kGgmlF32, {kHidden});
        require_tensor(file, p + "post_attention_norm.weight", kGgmlF32, {kHidden});
        require_tensor(file, p + "attn_q.weight", kGgmlQ8_0, {kHidden, kQueryWidth});
        require_tensor(file, p + "attn_q.bias", kGgmlF32, {kQueryWidth});
        require_tensor(file, p + "attn_k.weight", kGgmlQ8_0, {kHidden, kKvWidth});
        require_tensor(file, p + "attn_k.bias", kGgmlF32, {kKvWidth});
        require_tensor(file, p + "attn_v.weight", kGgmlQ8_0, {kHidden, kKvWidth});
        require_tensor(file, p + "attn_v.bias", kGgmlF32, {kKvWidth});
        require_tensor(file, p + "attn_output.weight", kGgmlQ8_0, {kQueryWidth, kHidden});
        require_tensor(file, p + "attn_output.bias", kGgmlF32, {kHidden});
        require_tensor(file, p + "attn_sinks.weight", kGgmlF32, {HipGptOssModel::query_heads});
        require_tensor(file, p + "ffn_gate_inp.weight", kGgmlF32, {kHidden, experts});
        require_tensor(file, p + "ffn_gate_inp.bias", kGgmlF32, {experts});
        require_tensor(file, p + "ffn_gate_exps.weight", kGgmlMxfp4, {kHidden, kHidden, experts});
        require_tensor(file, p + "ffn_gate_exps.bias", kGgmlF32, {kHidden, experts});
        require_tensor(file, p + "ffn_up_exps.weight", kGgmlMxfp4, {kHidden, kHidden, experts});
        require_tensor(file, p + "ffn_up_exps.bias", kGgmlF32, {kHidden, experts});
        require_tensor(file, p + "ffn_down_exps.weight", kGgmlMxfp4, {kHidden, kHidden, experts});
        require_tensor(file, p + "ffn_down_exps.bias", kGgmlF32, {kHidden, experts});
    }
    return shape;
}

void HipGptOssModel::upload_gguf(const GgufSource &file) {
    const uint32_t E = spec_.experts;
    auto f32 = [&](const std::string &name) {
        const TensorRef t = checked_tensor(file, name);
        float *p = static_cast<float *>(alloc(t.bytes));
        check(ttl_memcpy_h2d(ctx_, p, t.data, t.bytes), "ttl_memcpy_h2d");
        return p;
    };
    auto q8 = [&](const void *gguf_rows, uint32_t rows, uint32_t cols, const int32_t *row_source,
                  uint32_t source_rows) {
        ttl_q8 *t = nullptr;
        check(ttl_q8_upload(ctx_, gguf_rows, rows, cols, row_source, source_rows, &t), "ttl_q8_upload");
        device_bytes_ += ttl_q8_bytes(t);
        return t;
    };
    auto mxfp4 = [&](const std::string &name) {
        ttl_mxfp4 *t = nullptr;
        check(ttl_mxfp4_upload(ctx_, checked_tensor(file, name).data, uint32_t(kHidden), uint32_t(kHidden), E, &t),
              "ttl_mxfp4_upload");
        device_bytes_ += ttl_mxfp4_bytes(t);
        return t;
    };

    std::vector<int32_t> qkv_rows(kQkvRows);
    check(ttl_qkv_row_source(qkv_rows.data()), "ttl_qkv_row_source");
    const size_t q8_row = kHidden / 32 * 34;
    std::vector<uint8_t> qkv(kQkvRows * q8_row);  // attn_q | attn_k | attn_v rows, GGUF bytes
    std::vector<float> qkv_bias(kQkvRows);
    layers_.resize(spec_.layers);
    for (size_t i = 0; i < spec_.layers; ++i) {
        const std::string p = layer_prefix(i);
        Layer &layer = layers_[i];
        layer.attn_norm = f32(p + "attn_norm.weight");
        layer.post_norm = f32(p + "post_attention_norm.weight");
        size_t at = 0, bat = 0;
        for (const char *part : {"attn_q", "attn_k", "attn_v"}) {
            const TensorRef w = checked_tensor(file, p + part + ".weight");
            const TensorRef b = checked_tensor(file, p + part + ".bias");
            std::memcpy(qkv.data() + at, w.data, w.bytes);
            std::memcpy(qkv_bias.data() + bat, b.data, b.bytes);
            at += w.bytes;
            bat += b.bytes / sizeof(float);
        }
        layer.qkv = q8(qkv.data(), uint32_t(kQkvRows), uint32_t(kHidden), qkv_rows.data(), uint32_t(kQkvRows));
        layer.qkv_bias = static_cast<float *>(alloc(sizeof(float) * kQkvRows));
        check(ttl_memcpy_h2d(ctx_, layer.qkv_bias, qkv_bias.data(), sizeof(float) * kQkvRows), "ttl_memcpy_h2d");
        layer.attn_output = q8(checked_tensor(file, p + "attn_output.weight").data, uint32_t(kHidden),
                               uint32_t(kQueryWidth), nullptr, uint32_t(kHidden));
        layer.attn_output_bias = f32(p + "attn_output.bias");
        layer.sinks = f32(p + "attn_sinks.weight");
        layer.router = f32(p + "ffn_gate_inp.weight");
        layer.router_bias = f32(p + "ffn_gate_inp.bias");
        layer.gate = mxfp4(p + "ffn_gate_exps.weight");
        layer.up = mxfp4(p + "ffn_up_exps.weight");
        layer.down = mxfp4(p + "ffn_down_exps.weight");
        layer.gate_bias = f32(p + "ffn_gate_exps.bias");
        layer.up_bias = f32(p + "ffn_up_exps.bias");
        layer.down_bias = f32(p + "ffn_down_exps.bias");
        const size_t kv_bytes = sizeof(float) * spec_.capacity * kKvWidth;
        layer.key_cache = static_cast<float *>(alloc(kv_bytes));
        layer.value_cache = static_cast<float *>(alloc(kv_bytes));
        check(ttl_fill_bytes(ctx_, layer.key_cache, 0, kv_bytes), "fill");
        check(ttl_fill_bytes(ctx_, layer.value_cache, 0, kv_bytes), "fill");
        ttl_moe_layer &m = layer.moe;
        m.hidden = uint32_t(kHidden);
        m.expert_hidden = uint32_t(kHidden);
        m.experts = E;
        m.used = uint32_t(experts_used);
        m.router_weight = layer.router;
        m.router_bias = layer.router_bias;
        m.gate = layer.gate;
        m.gate_bias = layer.gate_bias;
        m.up = layer.up;
        m.up_bias = layer.up_bias;
        m.down = layer.down;
        m.down_bias = layer.down_bias;
        m.input_norm = layer.post_norm;  // model.cpp:590
        m.input_norm_epsilon = norm_epsilon;
    }
    const TensorRef embd = checked_tensor(file, "token_embd.weight");
    embedding_ = static_cast<uint8_t *>(alloc(embd.bytes));
    check(ttl_memcpy_h2d(ctx_, embedding_, embd.data, embd.bytes), "ttl_memcpy_h2d");
    output_norm_ = f32("output_norm.weight");
    const TensorRef out = checked_tensor(file, "output.weight");
    if (out.type == kGgmlBf16) {
        unembedding_ = static_cast<uint16_t *>(alloc(out.bytes));
        check(ttl_memcpy_h2d(ctx_, unembedding_, out.data, out.bytes), "ttl_memcpy_h2d");
    } else {
        unembedding_q8_ = q8(out.data, spec_.vocab, uint32_t(kHidden), nullptr, spec_.vocab);
    }
}

}  // namespace ttlab
