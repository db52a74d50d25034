// ref_gguf_dump.cpp -- the canonical dump (gguf_dump.hpp) of GGUF files as
// the reference's own reader and QwenConfig::from_gguf see them.
//
// TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile into oracle/_ref/ from
// the reference sources where they lie (src/io/gguf_reader.cpp,
// src/model/qwen_config.cpp, src/compute/common/dtype.cpp under REF_ROOT);
// nothing from the reference is copied into this repository.
//   ref_gguf_dump FILE...   one dump per file, each followed by a NUL line
#include "citlali/io/gguf_reader.h"
#include "citlali/model/qwen_config.h"
#include "gguf_dump.hpp"

#include <cstdio>

int main(int argc, char** argv) {
    for (int i = 1; i < argc; ++i) {
        const std::string d = gguf_dump::dump_path<citlali::io::GgufFile, citlali::model::QwenConfig>(
            argv[i], [](const citlali::io::GgufValue& v) { return citlali::io::metadata_value_to_string(v); });
        std::fwrite(d.data(), 1, d.size(), stdout);
        std::fputc('\0', stdout);
        std::fputc('\n', stdout);
    }
    return 0;
}
