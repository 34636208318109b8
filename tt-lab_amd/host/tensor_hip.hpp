// ttlab::HipTensorBackend -- the reference's tensor functions (tensor.h:18-51) on the
// gfx950 backend, for a caller that keeps the reference's GptOssModel and sends it the
// matrix work.  Same function names, argument meaning (shape[0] = inputs, shape[1] =
// outputs, shape[2] = experts, tensor.h:15-17) and error convention
// (std::runtime_error); host arrays in and out, as in the reference.
//
// The tensor arguments may be any descriptor laid out as the reference's GgufTensor
// (gguf.h:38-44: name, shape, type, data) -- the reference's own struct or
// ttlab::GgufTensorInfo -- so the reference's tensor.cpp can forward its calls here
// unchanged.  Each tensor goes to the device on first use and stays there (MXFP4 and
// Q8_0 repacked on the device, F32 as is), keyed by the address of its bytes, its
// byte count, type, shape and a fingerprint of about 2 KB sampled from its bytes on
// every call: a file mapped later at the same address with other weights there is
// uploaded again.  release_tensors() frees every device copy (the sure way, for a
// backend that outlives the file holding its tensors).
// Every call copies its input in and its output back and waits for it, so each pays a
// PCIe round trip: the whole-model facade (HipGptOssModel) keeps activations on the
// device instead.  Host code only: the device is reached through include/ttlab_hip.h.
#pragma once

#include "gguf_source.hpp"
#include "ttlab_hip.h"

#include <cstddef>
#include <cstdint>
#include <unordered_map>

namespace ttlab {

class HipTensorBackend {
  public:
    explicit HipTensorBackend(int device = 0);
    ~HipTensorBackend();
    HipTensorBackend(const HipTensorBackend &) = delete;
    HipTensorBackend &operator=(const HipTensorBackend &) = delete;

    // tensor.h:23, tensor.cpp:171-184: row `row` of a Q8_0 table.
    template <class T>
    void load_token_embedding_q8_0(const T &tensor, size_t row, float *output) {
        load_token_embedding_q8_0_ref(tensor_ref(tensor), row, output);
    }
    // tensor.h:24, tensor.cpp:186-200: output = bias + matrix input, each row summed in
    // the reference's sequential f32 order (the router's exact path), so the result is
    // the reference's bit for bit.  2880 inputs, at most 192 rows.
    template <class T>
    void matvec_add_f32(const T &matrix, const T &bias, const float *input, float *output) {
        matvec_add_f32_ref(tensor_ref(matrix), tensor_ref(bias), input, output);
    }
    // tensor.h:25-27, tensor.cpp:202-237.  2880 or 4096 inputs, rows a multiple of 16.
    template <class T>
    void matvec_q8_0(const T &matrix, const float *input, float *output) {
        matvec_q8_0_ref(tensor_ref(matrix), nullptr, input, output);
    }
    template <class T>
    void matvec_add_q8_0(const T &matrix, const T &bias, const float *input, float *output) {
        const TensorRef b = tensor_ref(bias);
        matvec_q8_0_ref(tensor_ref(matrix), &b, input, output);
    }
    // tensor.h:28-35, tensor.cpp:239-304: expert `expert` of a {2880, rows, experts}
    // MXFP4 tensor; bias f32 {rows, experts}.
    template <class T>
    void matvec_add_mxfp4_2880(const T &matrix, const T &bias, const float *input, float *output,
                               size_t expert = 0) {
        matvec_add_mxfp4_2880_ref(tensor_ref(matrix), tensor_ref(bias), input, output, expert);
    }
    // tensor.h:38-41, tensor.cpp:306-317, as the reference: transposed_input[c * count + s]
    // = input[tokens[s] * columns + c].
    template <class T>
    void transpose_selected(const T &matrix, const float *input, const size_t *tokens, size_t selected_count,
                            float *transposed_input) {
        transpose_selected_ref(tensor_ref(matrix), input, tokens, selected_count, transposed_input);
    }
    // tensor.h:42-51, tensor.cpp:319-495: output[tokens[s] * rows + r] for s <
    // selected_count; other rows of output are untouched.  `workspace` is the
    // reference's scratch and is not used (the device has its own).
    template <class T>
    void matmul_add_mxfp4_selected_transposed(const T &matrix, const T &bias, const float *transposed_input,
                                              const size_t *tokens, size_t selected_count, float *output,
                                              float *workspace, size_t expert = 0) {
        matmul_add_mxfp4_selected_transposed_ref(tensor_ref(matrix), tensor_ref(bias), transposed_input, tokens,
                                                 selected_count, output, workspace, expert);
    }
    // tensor.h:52, tensor.cpp:568-580, for the 2880-wide vectors of the model.
    template <class T>
    void rms_norm(const float *input, const T &weights, float epsilon, float *output) {
        rms_norm_ref(input, tensor_ref(weights), epsilon, output);
    }

    // Frees every tensor's device copy; later calls upload them again.
    void release_tensors();
    // Tensors held on the device.
    size_t resident_tensors() const {
        return mxfp4_.size() + q8_.size() + f32_.size();
    }

    ttl_ctx *context() const {
        return ctx_;
    }

  private:
    struct Buffer {
        void *dev = nullptr;
        size_t bytes = 0;
    };
    // What identifies a tensor's bytes: where they are, how many, and how they are read.
    struct Key {
        const void *data = nullptr;
        size_t bytes = 0;
        uint32_t type = 0;
        uint32_t dims = 0;
        uint64_t shape[4] = {0, 0, 0, 0};
        uint64_t fingerprint = 0;  // FNV-1a over samples of the bytes
        bool operator==(const Key &o) const;
    };
    struct KeyHash {
        size_t operator()(const Key &k) const;
    };
    static Key key_of(const TensorRef &t);

    void load_token_embedding_q8_0_ref(const TensorRef &tensor, size_t row, float *output);
    void matvec_add_f32_ref(const TensorRef &matrix, const TensorRef &bias, const float *input, float *output);
    void matvec_q8_0_ref(const TensorRef &matrix, const TensorRef *bias, const float *input, float *output);
    void matvec_add_mxfp4_2880_ref(const TensorRef &matrix, const TensorRef &bias, const float *input, float *output,
                                   size_t expert);
    void transpose_selected_ref(const TensorRef &matrix, const float *input, const size_t *tokens,
                                size_t selected_count, float *transposed_input);
    void matmul_add_mxfp4_selected_transposed_ref(const TensorRef &matrix, const TensorRef &bias,
                                                  const float *transposed_input, const size_t *tokens,
                                                  size_t selected_count, float *output, float *workspace,
                                                  size_t expert);
    void rms_norm_ref(const float *input, const TensorRef &weights, float epsilon, float *output);

    void *reserve(Buffer &buffer, size_t bytes);
    const ttl_mxfp4 *mxfp4_tensor(const TensorRef &tensor);
    const ttl_q8 *q8_tensor(const TensorRef &tensor);
    const float *f32_tensor(const TensorRef &tensor);

    ttl_ctx *ctx_ = nullptr;
    std::unordered_map<Key, ttl_mxfp4 *, KeyHash> mxfp4_;
    std::unordered_map<Key, ttl_q8 *, KeyHash> q8_;
    std::unordered_map<Key, void *, KeyHash> f32_;
    Buffer input_, output_, tokens_, workspace_, scratch_;
};

}  // namespace ttlab
