// The reference's tensor functions on the gfx950 backend (see tensor_hip.hpp).
#include "tensor_hip.hpp"

#include "gguf.hpp"        // GGML type ids
#include "gpt_oss_hip.hpp"  // ttlab::check

#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

namespace ttlab {
namespace {

void require(bool ok, const std::string &message) {
    if (!ok) {
        throw std::runtime_error(message);
    }
}

}  // namespace

bool HipTensorBackend::Key::operator==(const Key &o) const {
    if (data != o.data || bytes != o.bytes || type != o.type || dims != o.dims || fingerprint != o.fingerprint) {
        return false;
    }
    for (size_t d = 0; d < 4; ++d) {
        if (shape[d] != o.shape[d]) {
            return false;
        }
    }
    return true;
}

size_t HipTensorBackend::KeyHash::operator()(const Key &k) const {
    size_t h = std::hash<const void *>()(k.data);
    for (uint64_t v : {uint64_t(k.bytes), uint64_t(k.type), uint64_t(k.dims), k.shape[0], k.shape[1], k.shape[2],
                       k.shape[3], k.fingerprint}) {
        h ^= std::hash<uint64_t>()(v) + 0x9e3779b97f4a7c15ull + (h << 6) + (h >> 2);
    }
    return h;
}

HipTensorBackend::Key HipTensorBackend::key_of(const TensorRef &t) {
    Key k;
    k.data = t.data;
    k.bytes = t.bytes;
    k.type = t.type;
    k.dims = uint32_t(t.dims);
    for (size_t d = 0; d < t.dims && d < 4; ++d) {
        k.shape[d] = t.shape[d];
    }
    // the first and last 256 bytes and 16 evenly spaced runs of 64
    const auto *b = static_cast<const uint8_t *>(t.data);
    uint64_t h = 0xcbf29ce484222325ull;
    auto mix = [&](size_t at, size_t n) {
        for (size_t i = at; i < at + n && i < t.bytes; ++i) {
            h = (h ^ b[i]) * 0x100000001b3ull;
        }
    };
    if (b && t.bytes) {
        mix(0, 256);
        mix(t.bytes > 256 ? t.bytes - 256 : 0, 256);
        for (size_t i = 1; i < 16; ++i) {
            mix(t.bytes / 16 * i, 64);
        }
    }
    k.fingerprint = h;
    return k;
}

HipTensorBackend::HipTensorBackend(int device) {
    check(ttl_create(device, &ctx_), "ttl_create");
}

HipTensorBackend::~HipTensorBackend() {
    if (!ctx_) {
        return;
    }
    (void)ttl_sync(ctx_);
    release_tensors();
    for (Buffer *b : {&input_, &output_, &tokens_, &workspace_, &scratch_}) {
        if (b->dev) {
            (void)ttl_free(ctx_, b->dev);
        }
    }
    ttl_destroy(ctx_);
}

void HipTensorBackend::release_tensors() {
    (void)ttl_sync(ctx_);
    for (auto &entry : mxfp4_) {
        ttl_mxfp4_free(ctx_, entry.second);
    }
    for (auto &entry : q8_) {
        ttl_q8_free(ctx_, entry.second);
    }
    for (auto &entry : f32_) {
        (void)ttl_free(ctx_, entry.second);
    }
    mxfp4_.clear();
    q8_.clear();
    f32_.clear();
}

void *HipTensorBackend::reserve(Buffer &buffer, size_t bytes) {
    if (bytes > buffer.bytes) {
        if (buffer.dev) {
            check(ttl_sync(ctx_), "ttl_sync");
            check(ttl_free(ctx_, buffer.dev), "ttl_free");
            buffer.dev = nullptr;
            buffer.bytes = 0;
        }
        const size_t rounded = (bytes + 4095) / 4096 * 4096;
        check(ttl_malloc(ctx_, rounded, &buffer.dev), "ttl_malloc");
        buffer.bytes = rounded;
    }
    return buffer.dev;
}

const ttl_mxfp4 *HipTensorBackend::mxfp4_tensor(const TensorRef &t) {
    const Key key = key_of(t);
    const auto it = mxfp4_.find(key);
    if (it != mxfp4_.end()) {
        return it->second;
    }
    require(t.type == kGgmlMxfp4, "tensor " + std::string(t.name) + " is not MXFP4");
    ttl_mxfp4 *tensor = nullptr;
    check(ttl_mxfp4_upload(ctx_, t.data, uint32_t(t.extent(1)), uint32_t(t.extent(0)), uint32_t(t.extent(2)),
                           &tensor),
          "ttl_mxfp4_upload");
    mxfp4_.emplace(key, tensor);
    return tensor;
}

const ttl_q8 *HipTensorBackend::q8_tensor(const TensorRef &t) {
    const Key key = key_of(t);
    const auto it = q8_.find(key);
    if (it != q8_.end()) {
        return it->second;
    }
    require(t.type == kGgmlQ8_0, "tensor " + std::string(t.name) + " is not Q8_0");
    const uint32_t rows = uint32_t(t.extent(1));
    ttl_q8 *tensor = nullptr;
    check(ttl_q8_upload(ctx_, t.data, rows, uint32_t(t.extent(0)), nullptr, rows, &tensor), "ttl_q8_upload");
    q8_.emplace(key, tensor);
    return tensor;
}

// The tensor's bytes as they are (F32 vectors and matrices, or a Q8_0 table).
const float *HipTensorBackend::f32_tensor(const TensorRef &t) {
    const Key key = key_of(t);
    const auto it = f32_.find(key);
    if (it != f32_.end()) {
        return static_cast<const float *>(it->second);
    }
    void *dev = nullptr;
    check(ttl_malloc(ctx_, t.bytes, &dev), "ttl_malloc");
    const int rc = ttl_memcpy_h2d(ctx_, dev, t.data, t.bytes);
    if (rc != TTL_OK) {
        (void)ttl_free(ctx_, dev);
        check(rc, "ttl_memcpy_h2d");
    }
    f32_.emplace(key, dev);
    return static_cast<const float *>(dev);
}

void HipTensorBackend::load_token_embedding_q8_0_ref(const TensorRef &tensor, size_t row, float *output) {
    require(tensor.type == kGgmlQ8_0, "tensor " + std::string(tensor.name) + " is not Q8_0");
    const size_t n = tensor.extent(0), vocab = tensor.extent(1);
    require(row < vocab, "load_token_embedding_q8_0: row out of range");
    const void *table = f32_tensor(tensor);
    const int32_t token = int32_t(row);
    auto *token_dev = static_cast<int32_t *>(reserve(tokens_, sizeof(int32_t)));
    auto *out = static_cast<float *>(reserve(output_, n * sizeof(float)));
    check(ttl_memcpy_h2d(ctx_, token_dev, &token, sizeof token), "ttl_memcpy_h2d");
    check(ttl_embedding_q8_0(ctx_, table, uint32_t(vocab), token_dev, out), "ttl_embedding_q8_0");
    check(ttl_memcpy_d2h(ctx_, output, out, n * sizeof(float)), "ttl_memcpy_d2h");
}

void HipTensorBackend::matvec_add_f32_ref(const TensorRef &matrix, const TensorRef &bias, const float *input,
                                          float *output) {
    require(matrix.type == kGgmlF32 && bias.type == kGgmlF32, "matvec_add_f32: tensors must be F32");
    const size_t columns = matrix.extent(0), rows = matrix.extent(1);
    const float *weight = f32_tensor(matrix), *bias_dev = f32_tensor(bias);
    auto *x = static_cast<float *>(reserve(input_, columns * sizeof(float)));
    auto *logits = static_cast<float *>(reserve(output_, rows * sizeof(float)));
    auto *pick = static_cast<uint8_t *>(reserve(scratch_, 256));
    check(ttl_memcpy_h2d(ctx_, x, input, columns * sizeof(float)), "ttl_memcpy_h2d");
    // the router's exact path: each row summed in the reference's order
    check(ttl_router_topk(ctx_, weight, bias_dev, uint32_t(rows), uint32_t(columns), x, 1, TTL_ROUTER_FORCE_EXACT,
                          logits, reinterpret_cast<int32_t *>(pick), reinterpret_cast<float *>(pick + 128)),
          "ttl_router_topk");
    check(ttl_memcpy_d2h(ctx_, output, logits, rows * sizeof(float)), "ttl_memcpy_d2h");
}

void HipTensorBackend::matvec_q8_0_ref(const TensorRef &matrix, const TensorRef *bias, const float *input,
                                       float *output) {
    const size_t columns = matrix.extent(0), rows = matrix.extent(1);
    const ttl_q8 *w = q8_tensor(matrix);
    const float *bias_dev = bias ? f32_tensor(*bias) : nullptr;
    auto *x = static_cast<float *>(reserve(input_, columns * sizeof(float)));
    auto *y = static_cast<float *>(reserve(output_, rows * sizeof(float)));
    check(ttl_memcpy_h2d(ctx_, x, input, columns * sizeof(float)), "ttl_memcpy_h2d");
    ttl_stage_input in{};
    in.base = x;
    check(ttl_matvec_q8_0(ctx_, w, bias_dev, &in, nullptr, y), "ttl_matvec_q8_0");
    check(ttl_memcpy_d2h(ctx_, output, y, rows * sizeof(float)), "ttl_memcpy_d2h");
}

void HipTensorBackend::matvec_add_mxfp4_2880_ref(const TensorRef &matrix, const TensorRef &bias, const float *input,
                                                 float *output, size_t expert) {
    const size_t columns = matrix.extent(0), rows = matrix.extent(1);
    require(expert < matrix.extent(2), "matvec_add_mxfp4_2880: expert out of range");
    const ttl_mxfp4 *w = mxfp4_tensor(matrix);
    const float *bias_dev = f32_tensor(bias);
    auto *x = static_cast<float *>(reserve(input_, columns * sizeof(float)));
    auto *y = static_cast<float *>(reserve(output_, rows * sizeof(float)));
    check(ttl_memcpy_h2d(ctx_, x, input, columns * sizeof(float)), "ttl_memcpy_h2d");
    check(ttl_matvec_mxfp4(ctx_, w, bias_dev, x, y, uint32_t(expert)), "ttl_matvec_mxfp4");
    check(ttl_memcpy_d2h(ctx_, output, y, rows * sizeof(float)), "ttl_memcpy_d2h");
}

void HipTensorBackend::transpose_selected_ref(const TensorRef &matrix, const float *input, const size_t *tokens,
                                              size_t selected_count, float *transposed_input) {
    const size_t columns = matrix.extent(0);
    for (size_t s = 0; s < selected_count; ++s) {
        for (size_t c = 0; c < columns; ++c) {
            transposed_input[c * selected_count + s] = input[tokens[s] * columns + c];
        }
    }
}

void HipTensorBackend::matmul_add_mxfp4_selected_transposed_ref(const TensorRef &matrix, const TensorRef &bias,
                                                                const float *transposed_input, const size_t *tokens,
                                                                size_t selected_count, float *output,
                                                                float *workspace, size_t expert) {
    (void)workspace;
    if (selected_count == 0) {
        return;
    }
    const size_t columns = matrix.extent(0), rows = matrix.extent(1);
    require(expert < matrix.extent(2), "matmul_add_mxfp4_selected_transposed: expert out of range");
    const ttl_mxfp4 *w = mxfp4_tensor(matrix);
    const float *bias_dev = f32_tensor(bias);
    // the device reads token rows: undo the reference's transpose, rows in selection order
    std::vector<float> rows_in(selected_count * columns);
    for (size_t c = 0; c < columns; ++c) {
        for (size_t s = 0; s < selected_count; ++s) {
            rows_in[s * columns + c] = transposed_input[c * selected_count + s];
        }
    }
    std::vector<int32_t> order(selected_count);
    for (size_t s = 0; s < selected_count; ++s) {
        order[s] = int32_t(s);
    }
    const uint32_t count = uint32_t(selected_count);
    auto *x = static_cast<float *>(reserve(input_, rows_in.size() * sizeof(float)));
    auto *y = static_cast<float *>(reserve(output_, selected_count * rows * sizeof(float)));
    auto *tok = static_cast<int32_t *>(reserve(tokens_, selected_count * sizeof(int32_t)));
    const size_t ws_bytes = ttl_matmul_mxfp4_selected_workspace_bytes(count);
    void *ws = reserve(workspace_, ws_bytes);
    check(ttl_memcpy_h2d(ctx_, x, rows_in.data(), rows_in.size() * sizeof(float)), "ttl_memcpy_h2d");
    check(ttl_memcpy_h2d(ctx_, tok, order.data(), order.size() * sizeof(int32_t)), "ttl_memcpy_h2d");
    check(ttl_matmul_mxfp4_selected(ctx_, w, bias_dev, x, uint32_t(columns), count, tok, count, y, uint32_t(expert),
                                    ws, workspace_.bytes),
          "ttl_matmul_mxfp4_selected");
    std::vector<float> out(selected_count * rows);
    check(ttl_memcpy_d2h(ctx_, out.data(), y, out.size() * sizeof(float)), "ttl_memcpy_d2h");
    for (size_t s = 0; s < selected_count; ++s) {
        for (size_t r = 0; r < rows; ++r) {
            output[tokens[s] * rows + r] = out[s * rows + r];
        }
    }
}

void HipTensorBackend::rms_norm_ref(const float *input, const TensorRef &weights, float epsilon, float *output) {
    require(weights.type == kGgmlF32, "rms_norm: weights must be F32");
    const size_t n = weights.extent(0);
    require(n == 2880, "rms_norm: the device kernel takes vectors of 2880");
    const float *w = f32_tensor(weights);
    auto *x = static_cast<float *>(reserve(input_, n * sizeof(float)));
    auto *y = static_cast<float *>(reserve(output_, n * sizeof(float)));
    check(ttl_memcpy_h2d(ctx_, x, input, n * sizeof(float)), "ttl_memcpy_h2d");
    check(ttl_rms_norm_rows(ctx_, x, 1, w, epsilon, y), "ttl_rms_norm_rows");
    check(ttl_memcpy_d2h(ctx_, output, y, n * sizeof(float)), "ttl_memcpy_d2h");
}

}  // namespace ttlab
