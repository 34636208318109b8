// C API of ttlab::HipGptOssModel (include/ttlab_model.h): exceptions become status codes.
#include "gguf.hpp"
#include "gpt_oss_hip.hpp"
#include "tokenizer.hpp"
#include "ttlab_model.h"

#include <algorithm>
#include <cstring>
#include <exception>
#include <string>
#include <string_view>
#include <vector>

struct ttlm_model {
    ttlab::HipGptOssModel *model;
};

struct ttlm_tokenizer {
    ttlab::GgufFile file;  // the vocabulary and merges are views into its mapping
    ttlab::Tokenizer tokenizer;
    explicit ttlm_tokenizer(const char *path) : file(path), tokenizer(file) {}
};

namespace {

thread_local std::string last_error;

template <class F>
int guarded(F &&f) {
    try {
        f();
        return 0;
    } catch (const std::exception &e) {
        last_error = e.what();
    } catch (...) {
        last_error = "unknown error";
    }
    return -1;
}

}  // namespace

extern "C" {

const char *ttlm_last_error(void) {
    return last_error.c_str();
}

int ttlm_create_synthetic(int device, uint32_t layers, uint32_t experts, uint32_t vocab, uint32_t capacity,
                          uint64_t seed, ttlm_model **out) {
    if (!out) {
        last_error = "ttlm_create_synthetic: null output pointer";
        return -1;
    }
    *out = nullptr;
    return guarded([&] {
        ttlab::SyntheticSpec spec;
        spec.layers = layers;
        spec.experts = experts;
        spec.vocab = vocab;
        spec.capacity = capacity;
        spec.seed = seed;
        auto *m = new ttlab::HipGptOssModel(spec, device);
        *out = new ttlm_model{m};
    });
}

int ttlm_gguf_inspect(const char *path, int strict, ttlm_gguf_info *info) {
    return guarded([&] {
        if (!path || !info) {
            throw std::runtime_error("ttlm_gguf_inspect: null argument");
        }
        const ttlab::GgufFile file(path);
        const ttlab::GgufModelShape shape = ttlab::check_gguf_model(file, strict != 0);
        info->layers = shape.layers;
        info->experts = shape.experts;
        info->vocab = shape.vocab;
        info->output_type = shape.output_type;
        info->tensors = uint32_t(file.tensors().size());
    });
}

int ttlm_create_from_gguf(const char *path, int device, uint32_t capacity, int strict, ttlm_model **out) {
    if (!out) {
        last_error = "ttlm_create_from_gguf: null output pointer";
        return -1;
    }
    *out = nullptr;
    return guarded([&] {
        if (!path) {
            throw std::runtime_error("ttlm_create_from_gguf: null path");
        }
        const ttlab::GgufFile file(path);
        auto *m = new ttlab::HipGptOssModel(file, capacity, device, strict != 0);
        *out = new ttlm_model{m};
    });
}

void ttlm_destroy(ttlm_model *model) {
    if (model) {
        delete model->model;
        delete model;
    }
}

int ttlm_forward(ttlm_model *model, int32_t token, uint32_t position, float *logits) {
    return guarded([&] {
        const float *l = model->model->forward(token, position);
        if (logits) {
            std::memcpy(logits, l, sizeof(float) * model->model->spec().vocab);
        }
    });
}

int ttlm_prefill(ttlm_model *model, const int32_t *tokens, uint32_t count, float *logits) {
    return guarded([&] {
        const float *l = model->model->prefill(tokens, count);
        if (logits) {
            std::memcpy(logits, l, sizeof(float) * model->model->spec().vocab);
        }
    });
}

int ttlm_prefill_state(ttlm_model *model, uint32_t layer, uint32_t count, float *x_in) {
    return guarded([&] { model->model->prefill_state(layer, count, x_in); });
}

uint32_t ttlm_prefill_batch(const ttlm_model *model) {
    return uint32_t(model->model->prefill_batch());
}

int ttlm_generate(ttlm_model *model, int32_t token, uint32_t position, uint32_t steps, int32_t *tokens) {
    return guarded([&] {
        const std::vector<int32_t> out = model->model->generate(token, position, steps);
        if (tokens && !out.empty()) {
            std::memcpy(tokens, out.data(), sizeof(int32_t) * out.size());
        }
    });
}

int ttlm_time_decode(ttlm_model *model, int32_t token, uint32_t position, uint32_t warmup, uint32_t steps,
                     double *ms_per_step) {
    return guarded([&] { *ms_per_step = model->model->time_decode(token, position, warmup, steps); });
}

int ttlm_time_expert_kernel(ttlm_model *model, uint32_t reps, double *us_per_launch) {
    return guarded([&] { *us_per_launch = model->model->time_expert_kernel(reps); });
}

int ttlm_time_kernel(ttlm_model *model, uint32_t kind, uint32_t position, uint32_t reps, double *us_per_launch,
                     uint32_t *launches) {
    return guarded([&] {
        size_t n = 0;
        *us_per_launch = model->model->time_kernel(kind, position, reps, &n);
        if (launches) {
            *launches = uint32_t(n);
        }
    });
}

int ttlm_set_graph_replay(ttlm_model *model, int enabled) {
    return guarded([&] { model->model->set_graph_replay(enabled != 0); });
}

int ttlm_layer_state(ttlm_model *model, uint32_t layer, float *x_in, float *residual, int32_t *indices,
                     float *weights) {
    return guarded([&] { model->model->layer_state(layer, x_in, residual, indices, weights); });
}

int ttlm_final_state(ttlm_model *model, float *x_final) {
    return guarded([&] { model->model->final_state(x_final); });
}

int ttlm_kv_cache(ttlm_model *model, uint32_t layer, uint32_t positions, float *keys, float *values) {
    return guarded([&] { model->model->kv_cache(layer, positions, keys, values); });
}

int ttlm_fill_kv_synthetic(ttlm_model *model, uint32_t positions, uint64_t seed) {
    return guarded([&] { model->model->fill_kv_synthetic(positions, seed); });
}

size_t ttlm_device_bytes(const ttlm_model *model) {
    return model ? model->model->device_bytes() : 0;
}

double ttlm_step_bytes(const ttlm_model *model, uint32_t position) {
    return model ? model->model->step_bytes(position) : 0.0;
}

int ttlm_tokenizer_open(const char *gguf_path, ttlm_tokenizer **out) {
    if (!out || !gguf_path) {
        last_error = "ttlm_tokenizer_open: null argument";
        return -1;
    }
    *out = nullptr;
    return guarded([&] { *out = new ttlm_tokenizer(gguf_path); });
}

void ttlm_tokenizer_free(ttlm_tokenizer *tokenizer) {
    delete tokenizer;
}

int ttlm_tokenizer_encode(const ttlm_tokenizer *tokenizer, const char *text, size_t length, int32_t *tokens,
                          size_t capacity, size_t *count) {
    if (!tokenizer || (!text && length) || (!tokens && capacity) || !count) {
        last_error = "ttlm_tokenizer_encode: null argument";
        return -1;
    }
    return guarded([&] {
        const std::vector<int32_t> ids = tokenizer->tokenizer.encode(std::string_view(text ? text : "", length));
        *count = ids.size();
        std::memcpy(tokens, ids.data(), std::min(ids.size(), capacity) * sizeof(int32_t));
    });
}

int ttlm_tokenizer_decode(const ttlm_tokenizer *tokenizer, int32_t token, int render_special, char *out,
                          size_t capacity, size_t *written) {
    if (!tokenizer || (!out && capacity) || !written) {
        last_error = "ttlm_tokenizer_decode: null argument";
        return -1;
    }
    return guarded([&] { *written = tokenizer->tokenizer.decode_to(token, out, capacity, render_special != 0); });
}

size_t ttlm_tokenizer_vocabulary(const ttlm_tokenizer *tokenizer) {
    return tokenizer ? tokenizer->tokenizer.vocabulary_size() : 0;
}

int ttlm_pretokenize(const char *text, size_t length, size_t *ends, size_t capacity, size_t *count) {
    if ((!text && length) || (!ends && capacity) || !count) {
        last_error = "ttlm_pretokenize: null argument";
        return -1;
    }
    return guarded([&] {
        const std::string_view all(text ? text : "", length);
        const std::vector<std::string_view> pieces = ttlab::pretokenize(all);
        *count = pieces.size();
        for (size_t i = 0; i < pieces.size() && i < capacity; ++i) {
            ends[i] = size_t(pieces[i].data() - all.data()) + pieces[i].size();
        }
    });
}

size_t ttlm_harmony_prompt(const char *user, size_t length, char *out, size_t capacity) {
    const std::string formatted = ttlab::harmony_prompt(std::string_view(user ? user : "", user ? length : 0));
    if (out) {
        std::memcpy(out, formatted.data(), std::min(formatted.size(), capacity));
    }
    return formatted.size();
}

}  // extern "C"
