// ref_tok_dump.cpp -- the canonical dump (tok_dump.hpp) of the reference's
// own Tokenizer over GGUF files and a list of texts.
//
// TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile into oracle/_ref/ from
// the reference sources where they lie (src/tokenizer/tokenizer.cpp,
// src/io/gguf_reader.cpp, src/compute/common/dtype.cpp under REF_ROOT);
// nothing from the reference is copied into this repository.
//   ref_tok_dump TEXTS FILE...   one dump per file, each followed by a NUL line
//   ref_tok_dump --reload A B     tok_dump::reload of A then B
//   ref_tok_dump --fresh TEXTS    tok_dump::dump_fresh
#include "citlali/io/gguf_reader.h"
#include "citlali/tokenizer/tokenizer.h"
#include "tok_dump.hpp"

#include <cstdio>

int main(int argc, char** argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: ref_tok_dump TEXTS FILE...\n");
        return 2;
    }
    if (std::string(argv[1]) == "--fresh" && argc == 3) {
        const std::string d = tok_dump::dump_fresh<citlali::tokenizer::Tokenizer>(tok_dump::read_texts(argv[2]));
        std::fwrite(d.data(), 1, d.size(), stdout);
        return 0;
    }
    if (std::string(argv[1]) == "--reload" && argc == 4) {
        const std::string d = tok_dump::reload<citlali::io::GgufFile, citlali::tokenizer::Tokenizer>(argv[2], argv[3]);
        std::fwrite(d.data(), 1, d.size(), stdout);
        return 0;
    }
    const auto texts = tok_dump::read_texts(argv[1]);
    for (int i = 2; i < argc; ++i) {
        const std::string d = tok_dump::dump<citlali::io::GgufFile, citlali::tokenizer::Tokenizer>(argv[i], texts);
        std::fwrite(d.data(), 1, d.size(), stdout);
        std::fputc('\0', stdout);
        std::fputc('\n', stdout);
    }
    return 0;
}
