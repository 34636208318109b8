// ttlab_run: the reference CLI's generation path (main.cpp:275-411, `tt-lab run` and
// `tt-lab tokenize`) on the gfx950 backend.  The model, its checks, its decode loop and the
// tokenizer (ttlab::Tokenizer, the reference's Tokenizer restated) are the reference's.
//
//   ttlab_run run -m <model.gguf> (-p <prompt> | -t <id,id,...>) [-n <tokens>] [--device <ordinal>] [--loose]
//   ttlab_run tokenize -m <model.gguf> -p <text>
//   ttlab_run inspect -m <model.gguf> [--loose]
//
// `run -p` formats the prompt with the Harmony template (harmony_prompt), encodes it,
// prefills it, prints the formatted prompt and then each generated token's text, as the
// reference does; `run -t` takes the prompt as token ids and prints the generated ids.
// Generation follows the reference's greedy / forward loop (the forwards run on the device
// in chunks) until the end-of-sequence id (tokenizer.ggml.eos_token_id, required as in the
// reference) or the generation limit; the timing lines on stderr have the reference's
// format.  `tokenize` prints the ids of the text as the reference's does (no template).
// `inspect` applies the model checks (model.cpp:64-206) without a device and prints the
// shape it found.  Errors print "error: <message>" and exit 1, usage errors exit 2, as
// main.cpp does.  --loose admits the small test models (check_gguf_model(file, false)).
#include "gguf.hpp"
#include "gpt_oss_hip.hpp"
#include "tokenizer.hpp"

#include <algorithm>
#include <array>
#include <chrono>
#include <cstdio>
#include <iostream>
#include <limits>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

void usage(const char *argv0) {
    std::cerr << "usage: " << argv0
              << " run -m <model.gguf> (-p <prompt> | -t <id,id,...>) [-n <tokens>] [--device <ordinal>] [--loose]\n"
              << "       " << argv0 << " tokenize -m <model.gguf> -p <text>\n"
              << "       " << argv0 << " inspect -m <model.gguf> [--loose]\n";
}

bool parse_size(const std::string &text, size_t *output) {
    try {
        size_t used = 0;
        const unsigned long long parsed = std::stoull(text, &used);
        if (used != text.size() || text.empty() || text[0] == '-' ||
            parsed > std::numeric_limits<size_t>::max()) {
            return false;
        }
        *output = size_t(parsed);
        return true;
    } catch (const std::exception &) {
        return false;
    }
}

bool parse_tokens(const std::string &text, std::vector<int32_t> *tokens) {
    size_t start = 0;
    while (start <= text.size()) {
        const size_t comma = text.find(',', start);
        const std::string item = text.substr(start, comma == std::string::npos ? std::string::npos : comma - start);
        size_t value = 0;
        if (!parse_size(item, &value) || value > size_t(std::numeric_limits<int32_t>::max())) {
            return false;
        }
        tokens->push_back(int32_t(value));
        if (comma == std::string::npos) {
            break;
        }
        start = comma + 1;
    }
    return !tokens->empty();
}

double seconds(std::chrono::steady_clock::time_point begin, std::chrono::steady_clock::time_point end) {
    return std::chrono::duration<double>(end - begin).count();
}

}  // namespace

int main(int argc, char **argv) {
    if (argc < 2) {
        usage(argv[0]);
        return 2;
    }
    const std::string command = argv[1];
    if (command == "-h" || command == "--help") {
        usage(argv[0]);
        return 0;
    }
    if (command != "run" && command != "inspect" && command != "tokenize") {
        std::cerr << "unknown command: " << command << '\n';
        usage(argv[0]);
        return 2;
    }
    std::string model_path;
    std::vector<int32_t> prompt;
    bool tokens_set = false, predict_set = false, strict = true;
    const char *text = nullptr;
    size_t predict = 0, device = 0;
    for (int i = 2; i < argc; ++i) {
        const std::string argument = argv[i];
        if ((argument == "-m" || argument == "--model") && i + 1 < argc) {
            model_path = argv[++i];
        } else if ((argument == "-t" || argument == "--tokens") && i + 1 < argc) {
            if (!parse_tokens(argv[++i], &prompt)) {
                std::cerr << "invalid token list: " << argv[i] << '\n';
                return 2;
            }
            tokens_set = true;
        } else if ((argument == "-p" || argument == "--prompt") && i + 1 < argc) {
            text = argv[++i];
        } else if ((argument == "-n" || argument == "--predict" || argument == "--n-predict") && i + 1 < argc) {
            if (!parse_size(argv[++i], &predict)) {
                std::cerr << "invalid generation limit: " << argv[i] << '\n';
                return 2;
            }
            predict_set = true;
        } else if (argument == "--device" && i + 1 < argc) {
            if (!parse_size(argv[++i], &device) || device > 1024) {
                std::cerr << "invalid device ordinal: " << argv[i] << '\n';
                return 2;
            }
        } else if (argument == "--loose") {
            strict = false;
        } else {
            std::cerr << "unknown argument: " << argument << '\n';
            usage(argv[0]);
            return 2;
        }
    }
    if (model_path.empty() || (command == "run" && !tokens_set && !text) || (command == "tokenize" && !text)) {
        usage(argv[0]);
        return 2;
    }
    if (command == "run" && tokens_set && text) {
        std::cerr << "-p and -t are mutually exclusive\n";
        usage(argv[0]);
        return 2;
    }
    if (command != "run" && (tokens_set || predict_set)) {
        std::cerr << "-t and -n are only valid for 'run'\n";
        usage(argv[0]);
        return 2;
    }
    if (command == "inspect" && text) {
        std::cerr << "-p/--prompt is not valid for 'inspect'\n";
        usage(argv[0]);
        return 2;
    }

    try {
        const ttlab::GgufFile file(model_path);
        if (command == "tokenize") {
            // main.cpp:99-108, 286-289: the text's ids, without the chat template
            const ttlab::Tokenizer tokenizer(file);
            const std::vector<int32_t> ids = tokenizer.encode(text);
            std::cout << "prompt: " << text << "\ntokens (" << ids.size() << "): [";
            for (size_t k = 0; k < ids.size(); ++k) {
                std::cout << (k ? ", " : "") << ids[k];
            }
            std::cout << "]\n";
            return 0;
        }
        const ttlab::GgufModelShape shape = ttlab::check_gguf_model(file, strict);
        if (command == "inspect") {
            std::cout << "gpt-oss model: " << shape.layers << " layers, " << shape.experts
                      << " experts, vocabulary " << shape.vocab << ", output.weight type " << shape.output_type
                      << '\n';
            return 0;
        }
        // main.cpp:291-294: a text prompt in the Harmony template, encoded
        std::unique_ptr<ttlab::Tokenizer> tokenizer;
        std::string formatted;
        if (text) {
            tokenizer = std::make_unique<ttlab::Tokenizer>(file);
            formatted = ttlab::harmony_prompt(text);
            prompt = tokenizer->encode(formatted);
        }
        constexpr size_t context = ttlab::HipGptOssModel::context_length;
        if (prompt.size() > context) {
            throw std::runtime_error("prompt exceeds the model context");
        }
        const size_t limit = predict_set ? predict : context - prompt.size();
        if (limit > context - prompt.size()) {
            throw std::runtime_error("prompt and generation exceed the model context");
        }
        // main.cpp:373-411: the end-of-sequence id ends the generation; like the
        // reference, a file without the key is an error (GgufFile::integer throws)
        const int32_t eos = int32_t(file.integer("tokenizer.ggml.eos_token_id"));
        ttlab::HipGptOssModel model(file, prompt.size() + limit, int(device), strict);
        const auto prefill_begin = std::chrono::steady_clock::now();
        const float *logits = model.prefill(prompt.data(), prompt.size());
        const auto prefill_end = std::chrono::steady_clock::now();
        if (tokenizer) {
            std::cout << formatted << std::flush;
        }
        std::array<char, 8192> decoded;
        // The reference's loop (greedy, print, forward) with the forwards run on the device
        // in chunks: generate() feeds each step's argmax (the same first-maximum rule as
        // greedy) to the next step without a host round trip, and the chunk's tokens are
        // then printed, stopping at the end-of-sequence id as the reference does.  Steps a
        // chunk runs past that id are discarded and neither counted nor timed: each
        // counted forward adds its chunk's time divided by the chunk's steps.
        constexpr size_t kChunk = 32;
        std::vector<int32_t> pending{model.greedy(logits)};
        size_t next_index = 0, generated = 0, evaluations = 0;
        double decode_seconds = 0.0, step_seconds = 0.0;
        int32_t last = -1;
        for (size_t i = 0; i < limit; ++i) {
            if (next_index == pending.size()) {
                // token i follows token i - 1 at position prompt + i - 1
                const size_t steps = std::min(kChunk, limit - i);
                const auto begin = std::chrono::steady_clock::now();
                pending = model.generate(last, prompt.size() + i - 1, steps);
                step_seconds = seconds(begin, std::chrono::steady_clock::now()) / double(steps);
                next_index = 0;
            }
            const int32_t next = pending[next_index++];
            if (i > 0) {
                ++evaluations;  // the forward that produced this token (main.cpp counts it)
                decode_seconds += step_seconds;
            }
            if (next == eos) {
                break;
            }
            ++generated;
            if (tokenizer) {
                const size_t n = tokenizer->decode_to(next, decoded.data(), decoded.size(), true);
                std::cout.write(decoded.data(), std::streamsize(n));
                std::cout << std::flush;
            } else {
                std::cout << (generated > 1 ? " " : "") << next << std::flush;
            }
            last = next;
        }
        std::cout << '\n' << std::flush;
        const double prefill_seconds = seconds(prefill_begin, prefill_end);
        std::fprintf(stderr, "prefill: %zu tokens, %.3f s, %.3f t/s\n", prompt.size(), prefill_seconds,
                     double(prompt.size()) / prefill_seconds);
        std::fprintf(stderr, "generated: %zu tokens\n", generated);
        if (evaluations > 0) {
            std::fprintf(stderr, "decode: %zu evals, %.3f s, %.3f t/s\n", evaluations, decode_seconds,
                         double(evaluations) / decode_seconds);
        } else {
            std::fprintf(stderr, "decode: 0 evals, 0.000 s, n/a t/s\n");
        }
        return 0;
    } catch (const std::exception &error) {
        std::cerr << "error: " << error.what() << '\n';
        return 1;
    }
}
