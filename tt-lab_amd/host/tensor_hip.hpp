// ttlab::HipTensorBackend -- the reference's tensor functions (tensor.h:18-51) on the
// gfx950 backend, for a caller that keeps the reference's GptOssModel and sends it the
// matrix work.  Same function names, argument meaning (shape[0] = inputs, shape[1] =
// outputs, shape[2] = experts, tensor.h:15-17) and error convention
// (std::runtime_error); host arrays in and out, as in the reference.
//
// Each GGUF tensor goes to the device on first use, keyed by the address of its bytes
// in the mapped file, and stays there (MXFP4 and Q8_0 repacked on the device, F32 as
// is).  Every call copies its input in and its output back and waits for it, so each
// pays a PCIe round trip: the whole-model facade (HipGptOssModel) keeps activations
// on the device instead.  Host code only: the device is reached through
// include/ttlab_hip.h.
#pragma once

#include "gguf.hpp"
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
    void load_token_embedding_q8_0(const GgufTensorInfo &tensor, size_t row, float *output);
    // tensor.h:24, tensor.cpp:186-200: output = bias + matrix input, each row summed in
    // the reference's sequential f32 order (the router's exact path), so the result is
    // the reference's bit for bit.  2880 inputs, at most 192 rows.
    void matvec_add_f32(const GgufTensorInfo &matrix, const GgufTensorInfo &bias, const float *input, float *output);
    // tensor.h:25-27, tensor.cpp:202-237.  2880 or 4096 inputs, rows a multiple of 16.
    void matvec_q8_0(const GgufTensorInfo &matrix, const float *input, float *output);
    void matvec_add_q8_0(const GgufTensorInfo &matrix, const GgufTensorInfo &bias, const float *input,
                         float *output);
    // tensor.h:28-35, tensor.cpp:239-304: expert `expert` of a {2880, rows, experts}
    // MXFP4 tensor; bias f32 {rows, experts}.
    void matvec_add_mxfp4_2880(const GgufTensorInfo &matrix, const GgufTensorInfo &bias, const float *input,
                               float *output, size_t expert = 0);
    // tensor.h:38-41, tensor.cpp:306-317, as the reference: transposed_input[c * count + s]
    // = input[tokens[s] * columns + c].
    void transpose_selected(const GgufTensorInfo &matrix, const float *input, const size_t *tokens,
                            size_t selected_count, float *transposed_input);
    // tensor.h:42-51, tensor.cpp:319-495: output[tokens[s] * rows + r] for s <
    // selected_count; other rows of output are untouched.  `workspace` is the
    // reference's scratch and is not used (the device has its own).
    void matmul_add_mxfp4_selected_transposed(const GgufTensorInfo &matrix, const GgufTensorInfo &bias,
                                              const float *transposed_input, const size_t *tokens,
                                              size_t selected_count, float *output, float *workspace,
                                              size_t expert = 0);
    // tensor.h:52, tensor.cpp:568-580, for the 2880-wide vectors of the model.
    void rms_norm(const float *input, const GgufTensorInfo &weights, float epsilon, float *output);

    ttl_ctx *context() const {
        return ctx_;
    }

  private:
    struct Buffer {
        void *dev = nullptr;
        size_t bytes = 0;
    };
    void *reserve(Buffer &buffer, size_t bytes);
    const ttl_mxfp4 *mxfp4_tensor(const GgufTensorInfo &tensor);
    const ttl_q8 *q8_tensor(const GgufTensorInfo &tensor);
    const float *f32_tensor(const GgufTensorInfo &tensor);

    ttl_ctx *ctx_ = nullptr;
    std::unordered_map<const void *, ttl_mxfp4 *> mxfp4_;
    std::unordered_map<const void *, ttl_q8 *> q8_;
    std::unordered_map<const void *, void *> f32_;
    Buffer input_, output_, tokens_, workspace_, scratch_;
};

}  // namespace ttlab
