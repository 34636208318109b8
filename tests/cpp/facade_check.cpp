// A compiled caller of the two C++ facades, as the reference's own code would use them,
// through types shaped like the reference's (declared here, not taken from it):
//  - RefTensor has the members of the reference's GgufTensor (gguf.h:38-44: name,
//    shape, type, offset, const std::byte *data) and RefFile the accessors of its
//    GgufFile (gguf.h:67-72: find returning a pointer, tensor, string, integer,
//    number), so every facade call below binds as a reference call site would;
//  - ttlab::HipGptOssModel is built with the reference's constructor arguments
//    (model.h:19-20: file, token_capacity, dump_directory, batch_capacity, then the
//    backend's device and strictness) and driven like main.cpp:373-411 drives
//    GptOssModel (prefill, then greedy / forward until the generation limit), with the
//    reference's error convention (std::runtime_error, reported as "error: <message>");
//  - ttlab::HipTensorBackend called like tensor.h's functions (model.cpp's calls of
//    load_token_embedding_q8_0, rms_norm, matvec_add_q8_0, matvec_add_f32,
//    matvec_add_mxfp4_2880, transpose_selected + matmul_add_mxfp4_selected_transposed);
//    with --second, the backend then outlives the file and runs the same MXFP4 call on
//    a second file of the same shapes (its device copy must not be the first file's).
// Test infrastructure: tests/test_gpu_cpp_facade.py runs it on GGUF files it writes and
// checks every output file against the oracle and the ctypes path.
//
// usage: facade_check [--second <other.gguf>] <model.gguf> <out_dir> <generation_limit> <prompt token> ...
#include "gguf.hpp"
#include "gpt_oss_hip.hpp"
#include "tensor_hip.hpp"

#include <cmath>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <limits>
#include <memory>
#include <stdexcept>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace {

// A tensor descriptor with the reference's GgufTensor members.
struct RefTensor {
    std::string_view name;
    std::vector<uint64_t> shape;
    uint32_t type = 0;
    uint64_t offset = 0;
    const std::byte *data = nullptr;
};

// A metadata value as find() returns it (only its presence is used here).
struct RefValue {
    uint32_t type = 0;
};

// A GGUF file with the reference's GgufFile accessors, over ttlab's reader.
class RefFile {
  public:
    explicit RefFile(const char *path) : file_(path) {
        for (const ttlab::GgufTensorInfo &t : file_.tensors()) {
            RefTensor r;
            r.name = t.name;
            r.shape = t.shape;
            r.type = t.type;
            r.offset = t.offset;
            r.data = reinterpret_cast<const std::byte *>(t.data);
            tensors_.emplace(std::string(t.name), r);
        }
    }
    const RefValue *find(std::string_view key) const {
        const ttlab::GgufEntry *e = file_.find(key);
        if (!e) {
            return nullptr;
        }
        value_.type = uint32_t(e->kind);
        return &value_;
    }
    const RefTensor *tensor(std::string_view name) const {
        const auto it = tensors_.find(std::string(name));
        return it == tensors_.end() ? nullptr : &it->second;
    }
    std::string_view string(std::string_view key) const {
        return file_.string(key);
    }
    uint64_t integer(std::string_view key) const {
        return file_.integer(key);
    }
    double number(std::string_view key) const {
        return file_.number(key);
    }

  private:
    ttlab::GgufFile file_;
    std::unordered_map<std::string, RefTensor> tensors_;
    mutable RefValue value_;
};

void write_floats(const std::string &path, const float *data, size_t n) {
    std::ofstream out(path, std::ios::binary);
    out.write(reinterpret_cast<const char *>(data), std::streamsize(n * sizeof(float)));
    if (!out) {
        throw std::runtime_error("cannot write " + path);
    }
}

const RefTensor &tensor(const RefFile &file, const std::string &name) {
    const RefTensor *t = file.tensor(name);
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
    const char *second = nullptr;
    if (argc >= 3 && std::strcmp(argv[1], "--second") == 0) {
        second = argv[2];
        argc -= 2;
        argv += 2;
    }
    if (argc < 5) {
        std::cerr << "usage: facade_check [--second <other.gguf>] <model.gguf> <out_dir> <generation_limit> "
                     "<prompt token> ...\n";
        return 2;
    }
    try {
        const std::string dir = argv[2];
        const size_t generation_limit = size_t(std::strtoul(argv[3], nullptr, 10));
        std::vector<int32_t> prompt;
        for (int i = 4; i < argc; ++i) {
            prompt.push_back(int32_t(std::strtol(argv[i], nullptr, 10)));
        }
        auto opened = std::make_unique<RefFile>(argv[1]);
        const RefFile &file = *opened;
        const size_t vocab = size_t(tensor(file, "output.weight").shape[1]);

        // main.cpp:373-399: capacity = prompt + generation limit, prefill, then greedy
        // and forward until the limit (the test model's end-of-sequence id is outside
        // its vocabulary); the reference's constructor arguments, then the backend's
        // device and strictness (the test model is smaller than gpt-oss-20b)
        const size_t token_capacity = prompt.size() + generation_limit;
        ttlab::HipGptOssModel model(file, token_capacity, std::string(), prompt.size(), 0, /*strict=*/false);
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
        errors << message_of([&] { RefFile missing((dir + "/no-such-model.gguf").c_str()); }) << '\n';
        errors << message_of([&] { ttlab::HipGptOssModel dumping(file, token_capacity, dir, 0, 0, false); }) << '\n';
        errors << message_of([&] { ttlab::HipGptOssModel too_big(file, token_capacity, std::string(),
                                                                 token_capacity + 1, 0, false); })
               << '\n';

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

        if (second) {
            // the first file is closed while the backend keeps its device copies; the
            // second may be mapped where the first was
            const size_t resident = hip.resident_tensors();
            opened.reset();
            const RefFile other(second);
            std::vector<float> gated2(rows);
            hip.matvec_add_mxfp4_2880(tensor(other, "blk.0.ffn_gate_exps.weight"),
                                      tensor(other, "blk.0.ffn_gate_exps.bias"), normed.data(), gated2.data(), expert);
            write_floats(dir + "/mxfp4_second.f32", gated2.data(), rows);
            hip.release_tensors();
            std::cout << "facade_check: second file, " << resident << " tensors were resident, "
                      << hip.resident_tensors() << " after release\n";
        }
        std::cout << "facade_check: " << prompt.size() << " prompt tokens, " << generation_limit
                  << " generated, tensor calls done\n";
        return 0;
    } catch (const std::exception &error) {
        std::cerr << "error: " << error.what() << '\n';
        return 1;
    }
}
