// test_tokenizer.cpp -- the engine's Tokenizer behind tok_dump.hpp, and its
// merge loop timed on a long text.
//
//   test_tokenizer dump TEXTS FILE...   one dump per file, each followed by a
//                                       NUL line (the format of
//                                       oracle/_ref/ref_tok_dump)
//   test_tokenizer time FILE BYTES      encode a BYTES-long text built from
//                                       the vocabulary, print ms and tokens,
//                                       check decode(encode(text)) == text
//   test_tokenizer reload A B           tok_dump::reload of A then B
//   test_tokenizer fresh TEXTS          tok_dump::dump_fresh
// No GPU.
#include "citlali/common.h"
#include "citlali/io/gguf_reader.h"
#include "citlali/tokenizer/tokenizer.h"
#include "tok_dump.hpp"

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <string>

using citlali::io::GgufFile;
using citlali::tokenizer::Tokenizer;

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "";
    try {
        if (mode == "dump" && argc >= 3) {
            const auto texts = tok_dump::read_texts(argv[2]);
            for (int i = 3; i < argc; ++i) {
                const std::string d = tok_dump::dump<GgufFile, Tokenizer>(argv[i], texts);
                std::fwrite(d.data(), 1, d.size(), stdout);
                std::fputc('\0', stdout);
                std::fputc('\n', stdout);
            }
            return 0;
        }
        if (mode == "time" && argc == 4) {
            GgufFile g;
            g.load(argv[2]);
            Tokenizer t;
            t.load_from_gguf(g);
            const size_t bytes = std::strtoull(argv[3], nullptr, 10);
            std::string text;
            // pieces without '<', so that no control token is spelled across
            // two of them (control tokens decode to nothing)
            for (int32_t id = 0; text.size() < bytes; id = (id * 7 + 13) % t.vocab_size()) {
                const std::string piece = t.decode_token(id);
                if (piece.find('<') == std::string::npos) text += piece;
            }
            const auto t0 = std::chrono::steady_clock::now();
            const auto ids = t.encode(text, true);
            const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
            std::printf("encode %zu bytes -> %zu tokens in %.2f ms\n", text.size(), ids.size(), ms);
            citlali::require(t.decode(t.encode(text, false)) == text, "decode(encode(text)) == text");
            return 0;
        }
        if (mode == "fresh" && argc == 3) {
            const std::string d = tok_dump::dump_fresh<Tokenizer>(tok_dump::read_texts(argv[2]));
            std::fwrite(d.data(), 1, d.size(), stdout);
            return 0;
        }
        if (mode == "reload" && argc == 4) {
            const std::string d = tok_dump::reload<GgufFile, Tokenizer>(argv[2], argv[3]);
            std::fwrite(d.data(), 1, d.size(), stdout);
            return 0;
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
    std::fprintf(stderr, "usage: test_tokenizer dump TEXTS FILE... | time FILE BYTES | reload A B | fresh TEXTS\n");
    return 2;
}
