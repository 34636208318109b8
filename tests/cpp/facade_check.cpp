// A compiled caller of the two C++ facades, as the reference's own code would use them:
//  - ttlab::HipGptOssModel driven like main.cpp:373-411 drives GptOssModel (prefill,
//    then greedy / forward until the generation limit), with the reference's error
//    convention (std::runtime_error, reported as "error: <message>");
//  - ttlab::HipTensorBackend called like tensor.h's functions (model.cpp's calls of
//    load_token_embedding_q8_0, rms_norm, matvec_add_q8_0, matvec_add_f32,
//    matvec_add_mxfp4_2880, transpose_selected + matmul_add_mxfp4_selected_transposed).
// Test infrastructure: tests/test_gpu_cpp_facade.py runs it on a GGUF file it writes and
// checks every output file against the oracle and the ctypes path.
//
// usage: facade_check <model.gguf> <out_dir> <generation_limit> <prompt token> ...
#include "gguf.hpp"
#include "gpt_oss_hip.hpp"
#include "tensor_hip.hpp"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

void write_floats(const std::string &path, const float *data, size_t n) {
    std::ofstream out(path, std::ios::binary);
    out.write(reinterpret_cast<const char *>(data), std::streamsize(n * sizeof(float)));
    if (!out) {
        throw std::runtime_error("cannot write " + path);
    }
}

const ttlab::GgufTensorInfo &tensor(const ttlab::GgufFile &file, const std::string &name) {
    const ttlab::GgufTensorInfo *t = file.tensor(name);
    if (!t) {
        throw std::runtime_error("missing tensor " + name);
    }
    return *t;
}

// Runs `f`, which must throw std::runtime_error; returns its message.
template <class F>
std::string message_of(F &&f) {
    try {
        f();
    } catch (const std::runtime_error &error) {
        return error.what();
    }
    return "(no error)";
}

}  // namespace

int main(int argc, char **argv) {
    if (argc < 5) {
        std::cerr << "usage: facade_check <model.gguf> <out_dir> <generation_limit> <prompt token> ...\n";
        return 2;
    }
    try {
        const std::string dir = argv[2];
        const size_t generation_limit = size_t(std::strtoul(argv[3], nullptr, 10));
        std::vector<int32_t> prompt;
        for (int i = 4; i < argc; ++i) {
            prompt.push_back(int32_t(std::strtol(argv[i], nullptr, 10)));
        }
        ttlab::GgufFile file(argv[1]);
        const size_t vocab = size_t(tensor(file, "output.weight").shape[1]);

        // main.cpp:373-399: capacity = prompt + generation limit, prefill, then greedy
        // and forward until the limit (the test model has no EOS in its vocabulary)
        const size_t token_capacity = prompt.size() + generation_limit;
        ttlab::HipGptOssModel model(file, token_capacity, 0, /*strict=*/false);
        const float *logits = model.prefill(prompt.data(), prompt.size());
        std::ofstream tokens(dir + "/tokens.txt");
        for (size_t i = 0; i < generation_limit; ++i) {
            const int32_t next = model.greedy(logits);
            tokens << next << '\n';
            if (i + 1 < generation_limit) {
                logits = model.forward(next, prompt.size() + i);
            }
        }
        write_floats(dir + "/logits.f32", logits, vocab);

        // the reference's errors, caught as main.cpp:414-417 catches them
        std::ofstream errors(dir + "/errors.txt");
        errors << message_of([&] { model.forward(int32_t(vocab), 0); }) << '\n';
        errors << message_of([&] { model.forward(0, token_capacity); }) << '\n';
        const std::vector<int32_t> too_long(token_capacity + 1, 0);
        errors << message_of([&] { model.prefill(too_long.data(), too_long.size()); }) << '\n';
        errors << message_of([&] { model.prefill(prompt.data(), 0); }) << '\n';
        errors << message_of([&] { ttlab::GgufFile missing(dir + "/no-such-model.gguf"); }) << '\n';

        // tensor-level calls on layer 0's tensors
        ttlab::HipTensorBackend hip;
        const size_t n = 2880;
        std::vector<float> x(n), normed(n);
        hip.load_token_embedding_q8_0(tensor(file, "token_embd.weight"), size_t(prompt[0]), x.data());
        write_floats(dir + "/embedding.f32", x.data(), n);
        hip.rms_norm(x.data(), tensor(file, "blk.0.attn_norm.weight"), 1.0e-5f, normed.data());
        write_floats(dir + "/norm.f32", normed.data(), n);

        const auto &q = tensor(file, "blk.0.attn_q.weight");
        std::vector<float> query(size_t(q.shape[1]));
        hip.matvec_add_q8_0(q, tensor(file, "blk.0.attn_q.bias"), normed.data(), query.data());
        write_floats(dir + "/q8.f32", query.data(), query.size());

        const auto &router = tensor(file, "blk.0.ffn_gate_inp.weight");
        std::vector<float> router_logits(size_t(router.shape[1]));
        hip.matvec_add_f32(router, tensor(file, "blk.0.ffn_gate_inp.bias"), normed.data(), router_logits.data());
        write_floats(dir + "/router.f32", router_logits.data(), router_logits.size());

        const auto &gate = tensor(file, "blk.0.ffn_gate_exps.weight");
        const auto &gate_bias = tensor(file, "blk.0.ffn_gate_exps.bias");
        const size_t rows = size_t(gate.shape[1]), expert = size_t(gate.shape[2]) - 1;
        std::vector<float> gated(rows);
        hip.matvec_add_mxfp4_2880(gate, gate_bias, normed.data(), gated.data(), expert);
        write_floats(dir + "/mxfp4.f32", gated.data(), rows);

        // moe_batch's selected-token matmul (model.cpp:413-420): 6 token rows (the
        // embeddings of tokens 0..5), three of them selected out of order
        const size_t token_rows = 6;
        std::vector<float> inputs(token_rows * n);
        for (size_t t = 0; t < token_rows; ++t) {
            hip.load_token_embedding_q8_0(tensor(file, "token_embd.weight"), t, inputs.data() + t * n);
        }
        const size_t selected[3] = {5, 1, 3};
        std::vector<float> transposed(3 * n);
        hip.transpose_selected(gate, inputs.data(), selected, 3, transposed.data());
        std::vector<float> out(token_rows * rows, std::numeric_limits<float>::quiet_NaN());
        std::vector<float> workspace(64);
        hip.matmul_add_mxfp4_selected_transposed(gate, gate_bias, transposed.data(), selected, 3, out.data(),
                                                 workspace.data(), expert);
        write_floats(dir + "/selected.f32", out.data(), out.size());
        write_floats(dir + "/selected_inputs.f32", inputs.data(), inputs.size());
        std::cout << "facade_check: " << prompt.size() << " prompt tokens, " << generation_limit
                  << " generated, tensor calls done\n";
        return 0;
    } catch (const std::exception &error) {
        std::cerr << "error: " << error.what() << '\n';
        return 1;
    }
}
